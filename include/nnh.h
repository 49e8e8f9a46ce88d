/*
 * nnh.h - C ABI of the MI355X (gfx950) GEMM hot path for nn-cpp.
 *
 * Every entry point works on DEVICE pointers (hipMalloc'd or any device-accessible memory) and is
 * stream-ordered on `stream` (a hipStream_t passed as void*; NULL is the null stream). Nothing here
 * throws across the boundary: each call returns an nnh status code, and nnh_last_error() holds the
 * message of the calling thread's last failure. Shapes are validated on the host before anything is
 * launched; an invalid call launches nothing.
 *
 * Numerics: every GEMM-shaped result is bit-identical to nn-cpp's NN_NATIVE (AVX2/FMA) CPU build on
 * the same inputs: each output element is the reference's sequential fused multiply-add chain over the
 * depth, including its accumulate rule and its depth-cut rule. Results do not depend on stream, grid,
 * leading dimensions, alignment, batch size or concurrent launches, and repeat bit for bit.
 */
#ifndef NNH_H
#define NNH_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NNH_OK 0
#define NNH_ERR_INVALID 1  /* null pointer, leading dimension too small, size out of range */
#define NNH_ERR_SHAPE 2    /* non-conformable shapes: nn-cpp's TensorShapeError */
#define NNH_ERR_ALIAS 3    /* output overlaps an input (forbidden by include/nn/kernels/gemm.hpp:37-39) */
#define NNH_ERR_HIP 4      /* HIP runtime error (no device, launch failure, out of memory) */

#define NNH_MAX_BATCH_DIMS 4

/* Batch addressing for nnh_sgemm_batched: matrix (i0, .., i{ndim-1}) of A starts at
 * a + sum(i_d * stride_a[d]) (element strides; 0 broadcasts). Two levels express attention's
 * per-(sample, head) addressing (src/autograd/ops.cpp:1255-1256). ndim 0 means one matrix. */
typedef struct nnh_batch {
	int ndim;
	size_t shape[NNH_MAX_BATCH_DIMS];
	ptrdiff_t stride_a[NNH_MAX_BATCH_DIMS];
	ptrdiff_t stride_b[NNH_MAX_BATCH_DIMS];
	ptrdiff_t stride_c[NNH_MAX_BATCH_DIMS];
} nnh_batch;

#define NNH_BIAS_NONE 0
#define NNH_BIAS_COL 1 /* v += bias[col]: Linear (src/autograd/ops.cpp:726-730) */
#define NNH_BIAS_ROW 2 /* v += bias[row]: convolution's per-channel bias (ops.cpp:1396-1409) */

/* Applied to each finished C element: v = v + bias, then with relu: alive = v > 0, v = alive ? v : 0.
 * alive (optional) is one byte per C element, addressed like C. */
typedef struct nnh_epilogue {
	int bias_mode;
	int relu;
	const float* bias;
	unsigned char* alive;
} nnh_epilogue;

/* Message of the calling thread's last failed call ("" if none). */
const char* nnh_last_error(void);
/* Library version string. */
const char* nnh_version(void);

/*
 * C = op(A) op(B), or C += op(A) op(B) when accumulate; only the m x n region of C is written.
 * Replaces nn::kernels::sgemm (include/nn/kernels/gemm.hpp:57-59, src/kernels/gemm.cpp:546-556), same
 * argument meaning: A is m x k (stored k x m and read transposed when trans_a), B is k x n (stored
 * n x k when trans_b), row-major with leading dimensions lda, ldb, ldc. k == 0 zero-fills C (or leaves
 * it when accumulating); m == 0 or n == 0 touches nothing (gemm.cpp:344-350).
 */
int nnh_sgemm(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b,
              size_t ldb, float* c, size_t ldc, int accumulate, void* stream);

/*
 * A batch of nnh_sgemm products sharing m, n, k and leading dimensions, with an optional fused
 * epilogue (NULL: none). Replaces the per-matrix sgemm loops of Tensor matmul (src/tensor.cpp:616-640),
 * attention (ops.cpp:1252-1260) and convolution (ops.cpp:1390-1409); each matrix gets exactly the
 * bits a separate nn::kernels::sgemm call would give it.
 */
int nnh_sgemm_batched(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                      const float* b, size_t ldb, float* c, size_t ldc, int accumulate, const nnh_batch* batch,
                      const nnh_epilogue* epilogue, void* stream);

/* As nnh_sgemm_batched with a forced kernel tile configuration (0 .. nnh_gemm_config_count()-1, or -1
 * for the automatic choice). For tuning and for tests that show results do not depend on the tiling. */
int nnh_sgemm_config(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                     const float* b, size_t ldb, float* c, size_t ldc, int accumulate, const nnh_batch* batch,
                     const nnh_epilogue* epilogue, int config, void* stream);
int nnh_gemm_config_count(void);
const char* nnh_gemm_config_name(int config);

/*
 * Shape of nn::matmul(a, b, trans_a, trans_b) (src/tensor.cpp:571-641): NNH_ERR_SHAPE where the
 * reference throws TensorShapeError. out_shape needs room for max(a_ndim, b_ndim) entries.
 */
int nnh_matmul_shape(const size_t* a_shape, int a_ndim, const size_t* b_shape, int b_ndim, int trans_a,
                     int trans_b, size_t* out_shape, int* out_ndim);

/*
 * nn::matmul(a, b, trans_a, trans_b) on dense row-major device tensors (src/tensor.cpp:571-641): the
 * 2-D-right-operand fold into one GEMM (587-596) and leading-axis broadcasting (598-640) included.
 * out must hold the nnh_matmul_shape result.
 */
int nnh_matmul(const float* a, const size_t* a_shape, int a_ndim, const float* b, const size_t* b_shape, int b_ndim,
               int trans_a, int trans_b, float* out, void* stream);

/*
 * nn::linear forward (src/autograd/ops.cpp:714-730): y[M x n] = x[M x K] w[n x K]^T, then + bias[n] per
 * column, in one kernel. relu != 0 also applies the ReLU node that follows a Linear in the reference
 * (ops.cpp:775-782) in the same epilogue: y = v > 0 ? v : 0 (bit-identical to linear then relu).
 */
int nnh_linear_forward(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias, int relu,
                       float* y, void* stream);

/*
 * nn::linear backward (ops.cpp:731-744) for upstream gradient g of shape lead[0..nlead-1] x n, where x has
 * shape lead x K: dx = g w (sgemm F,F), dw = g^T x (sgemm T,F), db = g summed over every leading axis by
 * Tensor::sum(0), one axis at a time (ops.cpp:35-53). Each *_first selects nn-cpp's first-write rule for a
 * fresh gradient buffer (value.cpp:60-64): overwrite (db: s + 0.0f) instead of accumulate. Any of dx, dw,
 * db may be NULL (that input needs no gradient).
 */
int nnh_linear_backward(const float* g, const float* x, const float* w, const size_t* lead, int nlead, size_t K,
                        size_t n, float* dx, int dx_first, float* dw, int dw_first, float* db, int db_first,
                        void* stream);

/* nn::relu forward (ops.cpp:775-782): y = x > 0 ? x : 0. */
int nnh_relu_forward(const float* x, float* y, size_t count, void* stream);

/* nn::relu backward (ops.cpp:783-792): term = x > 0 ? g : 0; first: dx = term + 0.0f, else dx += term.
 * x may be the forward output instead of its input (y > 0 exactly where x > 0). */
int nnh_relu_backward(const float* x, const float* g, float* dx, int first, size_t count, void* stream);

/* Tensor::sum(0) of a {rows, inner} tensor (src/tensor.cpp:422-456): s_j = sum of src[a][j] over a in order,
 * from +0. combine 0: dst = s; 1: dst = s + 0.0f (a fresh gradient); 2: dst += s. */
int nnh_tensor_sum0(const float* src, size_t rows, size_t inner, float* dst, int combine, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NNH_H */
