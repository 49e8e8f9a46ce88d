/*
 * oracle.h - CPU restatement of nn-cpp's GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY. The product (nn-cpp_amd/) never links, loads or calls anything
 * here. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker.
 *
 * Two kinds of functions:
 *  - oracle_*      : bit-exact restatements of what nn-cpp computes when built with
 *                    NN_NATIVE on an AVX2/FMA host (file:line cited on each).
 *  - oracle_*_f64  : fp64 closed forms used for tolerance bounds and to pin the restatements.
 *
 * All matrices are row-major fp32; sizes and leading dimensions are size_t (as in the reference).
 */
#ifndef NNH_ORACLE_H
#define NNH_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- GEMM (include/nn/kernels/gemm.hpp:36-59, src/kernels/gemm.cpp) ---- */
void oracle_sgemm(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                  const float* b, size_t ldb, float* c, size_t ldc, int accumulate);
int oracle_depth_cut(size_t m, size_t n, size_t k);
size_t oracle_piece_depth(size_t m, size_t n, size_t k);
void oracle_set_numerics(int mode);
void oracle_sgemm_at(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                     const float* b, size_t ldb, int accumulate, const size_t* rows, const size_t* cols,
                     const float* c_old, size_t count, float* out);
void oracle_sgemm_naive(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                        const float* b, size_t ldb, float* c, size_t ldc, int accumulate);
void oracle_sgemm_f64(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                      const float* b, size_t ldb, const float* c_in, size_t ldc, int accumulate,
                      double* out, double* mag);

/* ---- reductions (src/tensor.cpp:422-456, src/autograd/ops.cpp:804-812) ---- */
void oracle_sum_axis0(const float* src, size_t rows, size_t inner, float* dst);
float oracle_lane_sum(const float* p, size_t n);

/* ---- linear (src/autograd/ops.cpp:714-745) ---- */
void oracle_linear_forward(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias,
                           float* y);
void oracle_linear_backward(const float* g, const float* x, const float* w, size_t M, size_t K, size_t n,
                            const size_t* lead, int nlead, float* dx, int dx_first, float* dw, int dw_first,
                            float* db, int db_first);
void oracle_relu(const float* x, float* y, size_t count);

/* ---- normalisation (src/autograd/ops.cpp:800-1078) ---- */
void oracle_batchnorm_forward(const float* x, size_t N, size_t C, size_t S, const float* w, const float* b, float eps,
                              int relu, float* y, unsigned char* alive, float* mean, float* var, float* inv_std);
void oracle_batchnorm_backward(const float* g, const float* x, const unsigned char* alive, const float* w,
                               const float* mean, const float* inv_std, size_t N, size_t C, size_t S, float* dx,
                               int dx_first, float* dw, int dw_first, float* db, int db_first);
void oracle_layernorm_forward(const float* x, size_t R, size_t D, const float* gm, const float* bt, float eps,
                              float* y, float* mean, float* inv_std);
void oracle_layernorm_backward(const float* g, const float* x, const float* gm, const float* mean,
                               const float* inv_std, size_t R, size_t D, float* dx, int dx_first, float* dgamma,
                               int dgamma_first, float* dbeta, int dbeta_first);
void oracle_batchnorm_f64(const float* x, size_t N, size_t C, size_t S, double eps, double* xhat);
void oracle_layernorm_f64(const float* x, size_t R, size_t D, double eps, double* xhat);

/* ---- element-wise (src/autograd/ops.cpp:451-481, 1991-2015; src/kernels/vmath.cpp) ---- */
float oracle_tanh_one(float x);
void oracle_gelu_forward(const float* x, size_t count, float* y, float* th);
void oracle_gelu_backward(const float* x, const float* th, const float* g, size_t count, float* dx, int first);
void oracle_embedding_backward(const float* g, const int32_t* rows, size_t count, size_t V, size_t D, float* dw,
                               int first);

/* ---- max pooling (src/autograd/ops.cpp:1609-1705) ---- */
void oracle_maxpool2d_forward(const float* x, size_t planes, size_t H, size_t W, size_t k, size_t s, float* y,
                              uint32_t* argmax);
void oracle_maxpool2d_backward(const float* g, const uint32_t* argmax, size_t planes, size_t H, size_t W, size_t k,
                               size_t s, float* dx, int first);

/* ---- convolution (src/autograd/ops.cpp:119-243, 1345-1472) ---- */
void oracle_conv2d_output_size(size_t h, size_t w, size_t kh, size_t kw, size_t stride, size_t padding,
                               size_t* h_out, size_t* w_out);
void oracle_im2col_sample(const float* x, float* col, size_t Cin, size_t H, size_t W, size_t kh, size_t kw,
                          size_t stride, size_t padding);
void oracle_col2im_sample_add(const float* col, float* x, size_t Cin, size_t H, size_t W, size_t kh,
                              size_t kw, size_t stride, size_t padding);
void oracle_conv2d_forward(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w,
                           size_t Cout, size_t kh, size_t kw, const float* bias, size_t stride, size_t padding,
                           int fuse_relu, float* y, unsigned char* alive);
void oracle_conv2d_backward(const float* g, const float* x, const float* w, const unsigned char* alive,
                            size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw,
                            size_t stride, size_t padding, float* dx, int dx_first, float* dw, float* db);
void oracle_conv2d_f64(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w, size_t Cout,
                       size_t kh, size_t kw, const float* bias, size_t stride, size_t padding, double* y,
                       double* mag);

/* ---- attention (src/autograd/ops.cpp:1169-1343) ---- */
void oracle_masked_softmax_row(const float* row, float* o, size_t Tk, size_t i, const float* ph, int causal,
                               float scale_by);
void oracle_masked_softmax_row_backward(const float* y, float* g, size_t Tk, size_t i, const float* ph,
                                        int causal, float scale_by);
void oracle_attention_forward(const float* q, const float* k, const float* v, size_t N, size_t Tq, size_t Tk,
                              size_t D, size_t heads, const float* pad, int causal, float* out, float* probs);
void oracle_attention_backward(const float* g, const float* q, const float* k, const float* v,
                               const float* probs, size_t N, size_t Tq, size_t Tk, size_t D, size_t heads,
                               const float* pad, int causal, float* dq, int dq_first, float* dk, int dk_first,
                               float* dv, int dv_first);
void oracle_scaled_masked_softmax_backward(const float* y, const float* g, size_t N, size_t H, size_t Tq, size_t Tk,
                                           float scale_by, const float* pad, int causal, float* dx, int first);
void oracle_scaled_masked_softmax(const float* x, size_t N, size_t H, size_t Tq, size_t Tk, float scale_by,
                                  const float* pad, int causal, float* y);
void oracle_attention_f64(const float* q, const float* k, const float* v, size_t N, size_t Tq, size_t Tk,
                          size_t D, size_t heads, const float* pad, int causal, double* out, double* probs);

/* ---- seeded inputs (apps/bench/runner.cpp:80-86: std::mt19937 + uniform_real_distribution<float>) ---- */
void oracle_mt19937_uniform(unsigned seed, float lo, float hi, float* out, size_t count);

#ifdef __cplusplus
}
#endif
#endif
