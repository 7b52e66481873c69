/*
 * qconv_oracle.h - CPU restatement of the reference's quantized NHWC convolution.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the HIP library is compared against;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product (libmiq_qconv) never links, calls or falls back to it.
 */
#ifndef QCONV_ORACLE_H_
#define QCONV_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* conv[7] = {pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, groups} */

/* Deterministic synthetic data: splitmix64 output number i of the stream `seed`. */
uint64_t orc_splitmix64(uint64_t seed, uint64_t i);
void orc_fill_i8_uniform(int8_t* out, int64_t count, uint64_t seed, int32_t lo, int32_t hi);
void orc_fill_i8_relu_half(int8_t* out, int64_t count, uint64_t seed);
void orc_fill_i32_uniform(int32_t* out, int64_t count, uint64_t seed, int32_t lo, int32_t hi);
void orc_fill_f32_uniform(float* out, int64_t count, uint64_t seed, float lo, float hi);

/* Output size with the rules of infer_conv_shape; 0 on success, -1 on a rejected shape. */
int orc_conv_output_shape(int32_t n, int32_t h, int32_t w, int32_t c, int32_t r, int32_t s, int32_t k,
                          const int32_t conv[7], int32_t* ho, int32_t* wo);

/* int32 accumulators on float codes with per-sample input zero points in_zp[n] and one
 * filter zero point; by = bx = 0 selects the plain KRSC filter, by, bx > 0 the blocked
 * [K, By, Bx, R, S, C/groups] filter.  Returns 0, or -1 on a rejected shape. */
int orc_conv_qi32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r,
                  int32_t s, int32_t k, const int32_t conv[7], const int32_t* in_zp, int32_t f_zp, int32_t by,
                  int32_t bx, int32_t* y);

/* int32 accumulators of int8 codes (zero points 0), on `nthreads` OpenMP threads
 * (<= 0: the OpenMP default). */
int orc_conv_i8_acc(const int8_t* x, int32_t n, int32_t h, int32_t w, int32_t c, const int8_t* wt, int32_t r,
                    int32_t s, int32_t k, const int32_t conv[7], int32_t* y, int32_t nthreads);

/* Requantization / dequantization of `npix` pixels x k channels of accumulators, with the
 * arithmetic defined in include/miq_qconv.h. bias may be NULL. */
void orc_requant_i8(const int32_t* acc, int64_t npix, int32_t k, const int32_t* bias, const float* w_scale,
                    float in_scale, float out_scale, int32_t relu, int8_t* y);
void orc_dequant_f32(const int32_t* acc, int64_t npix, int32_t k, const int32_t* bias, const float* w_scale,
                     float in_scale, float out_scale, int32_t relu, float* y);

/* fp32 convolution in the loop order and rounding of the reference's cpu_fprop_nhwc;
 * 0, or -1 on a rejected shape. */
int orc_conv_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r, int32_t s,
                 int32_t k, const int32_t conv[7], float* y, int32_t nthreads);

/* dx and dw of the fp32 convolution in the loop orders and rounding of the reference's
 * cpu_bprop_nhwc / cpu_grad_nhwc; dy is n x ho x wo x k; 0, or -1 on a rejected shape. */
int orc_bprop_f32(const float* dy, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r, int32_t s,
                  int32_t k, const int32_t conv[7], float* dx, int32_t nthreads);
int orc_grad_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* dy, int32_t r, int32_t s,
                 int32_t k, const int32_t conv[7], float* dw, int32_t nthreads);

/* Blocked (locally connected) fp32 convolution in the loop orders and rounding of the
 * reference's cpu_block_fprop_nhwc / cpu_block_bprop_nhwc / cpu_block_grad_nhwc: the output
 * grid splits into by x bx blocks of (ho/by) x (wo/bx) positions, each with its own filter
 * w[k][by][bx][r][s][c/groups].  bias / dbias are k*by*bx floats indexed [k][by][bx]
 * (bias_mode 0) or at [k][0][0] (bias_mode 1); either may be NULL.  0, or -1 on a rejected
 * shape. */
int orc_block_conv_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r,
                       int32_t s, int32_t k, const int32_t conv[7], int32_t by, int32_t bx, const float* bias,
                       int32_t bias_mode, float* y, int32_t nthreads);
int orc_block_bprop_f32(const float* dy, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r,
                        int32_t s, int32_t k, const int32_t conv[7], int32_t by, int32_t bx, float* dx,
                        int32_t nthreads);
int orc_block_grad_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* dy, int32_t r,
                       int32_t s, int32_t k, const int32_t conv[7], int32_t by, int32_t bx, float* dw, float* dbias,
                       int32_t bias_mode, int32_t nthreads);

/* The blocked bias gradient in the fixed order of this library's kernels: dy (n x ho x wo x k)
 * summed over every position of a block, in runs of `chunk` positions (<= 0: one run) added in
 * order; mode 0 per block, mode 1 into [k][0][0].  0, or -1 on a grid that does not divide. */
int orc_block_dbias_f32(const float* dy, int32_t n, int32_t ho_n, int32_t wo_n, int32_t k, int32_t by, int32_t bx,
                        int32_t mode, int32_t chunk, float* dbias);

/* int32 batched matrix product with wrap-around arithmetic, the semantics of the
 * reference's bmm_matmul_i32: A[b] M x K (stored K x M when trans_a), B[b] K x N (stored
 * N x K when trans_b), C[b] M x N, batch strides M*K, K*N, M*N. */
void orc_bmm_i32(const int32_t* A, const int32_t* B, int32_t* C, int32_t batch, int32_t M, int32_t N, int32_t K,
                 int32_t trans_a, int32_t trans_b, int32_t nthreads);

#ifdef __cplusplus
}
#endif

#endif /* QCONV_ORACLE_H_ */
