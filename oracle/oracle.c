/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY.  A plain-C restatement of miniTensor's
 * CPU reference path for the fp32 GEMM family, used as the checker for the
 * HIP library and as the timed CPU baseline.  Nothing in the product
 * (minitensor_amd/) links, loads or calls this file.
 *
 * Built with `gcc -O2 -ffp-contract=off` (oracle/Makefile) so that every
 * `sum += a*b` rounds the product and the sum separately, as the reference's
 * GCC build does (no FMA contraction without -march, ISO C++20 mode;
 * reference CMakeLists.txt:15-21).
 *
 * Functions and the reference code each one restates:
 *   ora_matmul          include/TensorOps.hpp:139-160  matmul_cpu (i->j->k, fp32 acc)
 *   ora_matmul_strided  include/TensorOps.hpp:162-189  matmul_cpu_strided
 *   ora_bmm             include/TensorOps.hpp:933-991  bmm's intent: matmul_cpu per batch
 *   ora_conv2d          include/TensorOps.hpp:235-273  conv2d_cpu (bias first, c_in->r->s)
 *   ora_conv2d_bwd_input  include/TensorOps.hpp:318-353  conv2d_backward_input_cpu (scatter order)
 *   ora_conv2d_bwd_weight include/TensorOps.hpp:355-394  conv2d_backward_weight_cpu (per-image sums)
 *   ora_conv2d_bwd_bias   include/TensorOps.hpp:396-415  conv2d_backward_bias_cpu (per-image sums)
 *   ora_colsum          include/TensorOps.hpp:190-233  sum_cpu over axis 0 (sequential)
 *   ora_matmul_f64_rows (checker) fp64 brute force of selected rows
 *   ora_mt19937_*, ora_fill_*  deterministic seeded inputs (std::mt19937 + own transforms)
 *
 * Pinning (tests/test_oracle.py): the reference's known-answer tests, a
 * build of the reference headers themselves (oracle/_ref), fp64 brute force,
 * and algebraic invariants.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* ---- std::mt19937 (Matsumoto & Nishimura 1998, as fixed by [rand.eng.mers]) ---- */
void ora_mt19937_seed(ora_mt19937* g, uint32_t seed) {
    g->s[0] = seed;
    for (int i = 1; i < 624; ++i)
        g->s[i] = 1812433253u * (g->s[i - 1] ^ (g->s[i - 1] >> 30)) + (uint32_t)i;
    g->i = 624;
}

uint32_t ora_mt19937_next(ora_mt19937* g) {
    if (g->i >= 624) {
        for (int k = 0; k < 624; ++k) {
            uint32_t y = (g->s[k] & 0x80000000u) | (g->s[(k + 1) % 624] & 0x7fffffffu);
            uint32_t v = g->s[(k + 397) % 624] ^ (y >> 1);
            if (y & 1u) v ^= 0x9908b0dfu;
            g->s[k] = v;
        }
        g->i = 0;
    }
    uint32_t y = g->s[g->i++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

/* u in [0,1) with 24 random bits: exactly representable in fp32. */
static double u01(ora_mt19937* g) { return (double)(ora_mt19937_next(g) >> 8) * (1.0 / 16777216.0); }

void ora_fill_uniform(float* out, size_t n, uint32_t seed, float lo, float hi) {
    ora_mt19937 g;
    ora_mt19937_seed(&g, seed);
    for (size_t i = 0; i < n; ++i) out[i] = (float)((double)lo + ((double)hi - (double)lo) * u01(&g));
}

/* Box-Muller: one normal from each pair of uniforms (the cosine branch). */
void ora_fill_normal(float* out, size_t n, uint32_t seed, float mean, float std) {
    ora_mt19937 g;
    ora_mt19937_seed(&g, seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; ++i) {
        const double a = 1.0 - u01(&g); /* (0, 1] */
        const double b = u01(&g);
        const double z = sqrt(-2.0 * log(a)) * cos(two_pi * b);
        out[i] = (float)((double)mean + (double)std * z);
    }
}

/* ---- GEMM family ---------------------------------------------------------------- */
void ora_matmul(const float* a, const float* b, float* c, size_t M, size_t K, size_t N) {
    for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) {
            float sum = 0.0f;
            for (size_t k = 0; k < K; ++k) sum += a[i * K + k] * b[k * N + j];
            c[i * N + j] = sum;
        }
}

void ora_matmul_strided(const float* a, size_t a_sm, size_t a_sk, const float* b, size_t b_sk,
                        size_t b_sn, float* c, size_t c_sm, size_t c_sn, size_t M, size_t K,
                        size_t N) {
    for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) {
            float sum = 0.0f;
            for (size_t k = 0; k < K; ++k) {
                const float av = a[i * a_sm + k * a_sk];
                const float bv = b[k * b_sk + j * b_sn];
                sum += av * bv;
            }
            c[i * c_sm + j * c_sn] = sum;
        }
}

void ora_bmm(const float* a, const float* b, float* c, size_t batch, size_t M, size_t K,
             size_t N) {
    for (size_t z = 0; z < batch; ++z) ora_matmul(a + z * M * K, b + z * K * N, c + z * M * N, M, K, N);
}

void ora_conv2d(const float* in, const float* w, const float* bias, float* out, size_t N,
                size_t C_in, size_t H, size_t W, size_t C_out, size_t kH, size_t kW,
                size_t stride, size_t pad) {
    const size_t H_out = (H + 2 * pad < kH) ? 0 : (H + 2 * pad - kH) / stride + 1;
    const size_t W_out = (W + 2 * pad < kW) ? 0 : (W + 2 * pad - kW) / stride + 1;
    for (size_t n = 0; n < N; ++n)
        for (size_t co = 0; co < C_out; ++co)
            for (size_t y = 0; y < H_out; ++y)
                for (size_t x = 0; x < W_out; ++x) {
                    float val = bias ? bias[co] : 0.0f;
                    for (size_t ci = 0; ci < C_in; ++ci)
                        for (size_t r = 0; r < kH; ++r)
                            for (size_t s = 0; s < kW; ++s) {
                                const long iy = (long)(y * stride + r) - (long)pad;
                                const long ix = (long)(x * stride + s) - (long)pad;
                                if (iy >= 0 && iy < (long)H && ix >= 0 && ix < (long)W) {
                                    const size_t ii = n * (C_in * H * W) + ci * (H * W) + (size_t)iy * W + (size_t)ix;
                                    const size_t wi = co * (C_in * kH * kW) + ci * (kH * kW) + r * kW + s;
                                    val += in[ii] * w[wi];
                                }
                            }
                    out[n * (C_out * H_out * W_out) + co * (H_out * W_out) + y * W_out + x] = val;
                }
}

static size_t out_dim(size_t in, size_t pad, size_t k, size_t stride) {
    return (in + 2 * pad < k) ? 0 : (in + 2 * pad - k) / stride + 1;
}

void ora_conv2d_bwd_input(const float* go, const float* w, float* gi, size_t N, size_t C_in,
                          size_t H, size_t W, size_t C_out, size_t kH, size_t kW, size_t stride,
                          size_t pad) {
    const size_t Ho = out_dim(H, pad, kH, stride), Wo = out_dim(W, pad, kW, stride);
    memset(gi, 0, N * C_in * H * W * sizeof(float));
    for (size_t n = 0; n < N; ++n)
        for (size_t co = 0; co < C_out; ++co)
            for (size_t y = 0; y < Ho; ++y)
                for (size_t x = 0; x < Wo; ++x) {
                    const float g = go[n * (C_out * Ho * Wo) + co * (Ho * Wo) + y * Wo + x];
                    for (size_t ci = 0; ci < C_in; ++ci)
                        for (size_t r = 0; r < kH; ++r)
                            for (size_t s = 0; s < kW; ++s) {
                                const long iy = (long)(y * stride + r) - (long)pad;
                                const long ix = (long)(x * stride + s) - (long)pad;
                                if (iy >= 0 && iy < (long)H && ix >= 0 && ix < (long)W)
                                    gi[n * (C_in * H * W) + ci * (H * W) + (size_t)iy * W + (size_t)ix] +=
                                        g * w[co * (C_in * kH * kW) + ci * (kH * kW) + r * kW + s];
                            }
                }
}

void ora_conv2d_bwd_weight(const float* go, const float* in, float* gw, size_t N, size_t C_in,
                           size_t H, size_t W, size_t C_out, size_t kH, size_t kW, size_t stride,
                           size_t pad) {
    const size_t Ho = out_dim(H, pad, kH, stride), Wo = out_dim(W, pad, kW, stride);
    memset(gw, 0, C_out * C_in * kH * kW * sizeof(float));
    for (size_t n = 0; n < N; ++n)
        for (size_t co = 0; co < C_out; ++co)
            for (size_t ci = 0; ci < C_in; ++ci)
                for (size_t r = 0; r < kH; ++r)
                    for (size_t s = 0; s < kW; ++s) {
                        float sum = 0.0f;
                        for (size_t y = 0; y < Ho; ++y)
                            for (size_t x = 0; x < Wo; ++x) {
                                const long iy = (long)(y * stride + r) - (long)pad;
                                const long ix = (long)(x * stride + s) - (long)pad;
                                if (iy >= 0 && iy < (long)H && ix >= 0 && ix < (long)W)
                                    sum += in[n * (C_in * H * W) + ci * (H * W) + (size_t)iy * W + (size_t)ix] *
                                           go[n * (C_out * Ho * Wo) + co * (Ho * Wo) + y * Wo + x];
                            }
                        gw[co * (C_in * kH * kW) + ci * (kH * kW) + r * kW + s] += sum;
                    }
}

void ora_conv2d_bwd_bias(const float* go, float* gb, size_t N, size_t C_out, size_t Ho, size_t Wo) {
    memset(gb, 0, C_out * sizeof(float));
    for (size_t n = 0; n < N; ++n)
        for (size_t c = 0; c < C_out; ++c) {
            float sum = 0.0f;
            for (size_t i = 0; i < Ho * Wo; ++i) sum += go[n * (C_out * Ho * Wo) + c * (Ho * Wo) + i];
            gb[c] += sum;
        }
}

void ora_colsum(const float* x, size_t rs, size_t cs, size_t R, size_t Cn, float* out) {
    for (size_t c = 0; c < Cn; ++c) {
        float sum = 0.0f;
        for (size_t r = 0; r < R; ++r) sum += x[r * rs + c * cs];
        out[c] = sum;
    }
}

/* ---- checkers ------------------------------------------------------------------- */
void ora_matmul_f64_rows(const float* a, size_t a_sm, size_t a_sk, const float* b, size_t b_sk,
                         size_t b_sn, const int64_t* rows, size_t n_rows, size_t K, size_t N,
                         double* out) {
    for (size_t t = 0; t < n_rows; ++t) {
        const size_t i = (size_t)rows[t];
        for (size_t j = 0; j < N; ++j) {
            double sum = 0.0;
            for (size_t k = 0; k < K; ++k) sum += (double)a[i * a_sm + k * a_sk] * (double)b[k * b_sk + j * b_sn];
            out[t * N + j] = sum;
        }
    }
}
