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
#define NNH_ERR_WORKSPACE 5 /* the caller registered a workspace for the stream that is smaller than the call needs */

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

/*
 * Scratch memory. Some calls need device scratch beyond their inputs and outputs (the partial sums of a depth cut
 * whose pieces are spread over workgroups, the convolution backward's masked gradient and per-sample sums,
 * attention's dS). Each (device, stream) pair has one
 * scratch buffer, used by the calls on that stream in turn. By default the library owns it: allocated on the first
 * call that needs it, grown on demand, kept until the process ends.
 *
 * nnh_set_workspace registers a caller-owned device buffer of `bytes` bytes as the scratch of every call on
 * `stream` (on the device the stream belongs to). After it, no call on that stream allocates device memory: a call
 * that needs more than `bytes` returns NNH_ERR_WORKSPACE before launching anything. The buffer must stay valid
 * until the work enqueued on the stream with it has finished. workspace NULL with bytes 0 gives the stream back to
 * the library's own buffer. There is no counterpart in the reference, whose only scratch is thread-local packing
 * buffers (src/kernels/gemm.cpp:354, 395, 416, 467).
 *
 * The *_workspace_size queries give, for the same shape arguments as the call, the bytes that call takes (at least
 * what it needs: where a kernel choice depends on pointer alignment, the larger of the two; over both numerics
 * modes, the larger of the two; nnh_conv2d_backward_workspace_size with with_alive = 1 also covers
 * nnh_conv2d_backward_packed). One exception: nnh_sgemm_workspace_size cannot see leading dimensions, and a
 * depth-cut product of at most 16 pieces called with lda or ldb of 2^24 or more needs pieces * m * n * batch_count
 * floats of partials that it does not count (with a registered workspace smaller than that, the call returns
 * NNH_ERR_WORKSPACE before launching anything).
 */
int nnh_set_workspace(void* stream, void* workspace, size_t bytes);
int nnh_sgemm_workspace_size(size_t m, size_t n, size_t k, size_t batch_count, size_t* bytes);
int nnh_matmul_workspace_size(const size_t* a_shape, int a_ndim, const size_t* b_shape, int b_ndim, int trans_a,
                              int trans_b, size_t* bytes);
int nnh_linear_forward_workspace_size(size_t M, size_t K, size_t n, size_t* bytes);
int nnh_linear_backward_workspace_size(const size_t* lead, int nlead, size_t K, size_t n, int want_dx, int want_dw,
                                       int want_db, size_t* bytes);
int nnh_conv2d_forward_workspace_size(size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw,
                                      int stride, int padding, size_t* bytes);
int nnh_conv2d_backward_workspace_size(size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw,
                                       int stride, int padding, int with_alive, int want_dx, int want_dw, int want_db,
                                       size_t* bytes);
int nnh_attention_forward_workspace_size(size_t N, size_t Tq, size_t Tk, size_t D, size_t heads, size_t* bytes);
int nnh_attention_backward_workspace_size(size_t N, size_t Tq, size_t Tk, size_t D, size_t heads, size_t* bytes);

/*
 * Numerics mode. NNH_NUMERICS_NNCPP (the default): every result is
 * nn-cpp's bits, as described above. NNH_NUMERICS_SPLIT_DEPTH: every product with m n <= 2^18 and k >= 256 is
 * computed the way nn-cpp's depth cut computes its products (src/kernels/gemm.cpp:453-485), fused multiply-add
 * chains from +0 over consecutive slices of the depth, added in slice order, then stored or added to C, with a
 * slice depth chosen so the product fills the GPU: with T = ceil(m / 64) ceil(n / 16) and s = min(16, max(2,
 * 4096 / T)), ceil(k / s) rounded up to a multiple of 32. Short chains let small and skinny products use the whole
 * GPU. Results stay deterministic, a pure function of (m, n, k) and the inputs (so fused ops still equal their
 * compositions), within 4 K 2^-24 sum|a||b| of the exact product, and equal to the oracle's in the same mode; they
 * are no longer nn-cpp's bits for the products the rule cuts differently from nn-cpp.
 */
#define NNH_NUMERICS_DEFAULT (-1)
#define NNH_NUMERICS_NNCPP 0
#define NNH_NUMERICS_SPLIT_DEPTH 1
/* The process default, for streams without a mode of their own (no counterpart in nn-cpp, which has one
 * arithmetic). */
int nnh_set_numerics(int mode);
int nnh_get_numerics(void);
/* A stream's own mode (NNH_NUMERICS_DEFAULT: back to the process default), so that callers in one process can run
 * different modes at once. A call reads its stream's mode once, when it enters the library, and runs wholly in it:
 * a mode set while another thread enqueues work takes effect from that thread's next call. The *_workspace_size
 * queries answer for both modes. */
int nnh_set_stream_numerics(void* stream, int mode);
int nnh_get_stream_numerics(void* stream);

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
 * Backward of nn::matmul(a, b) (b_transposed = 0, src/autograd/ops.cpp:683-712) and nn::matmul_bt(a, b)
 * (b_transposed = 1, ops.cpp:747-773) for upstream gradient g of the forward's output shape. With b a 2-D matrix,
 * a's leading axes fold into M rows and each gradient is one sgemm with accumulate = !first; otherwise the
 * gradient is a batched product reduced over broadcast axes (sum_to_shape, ops.cpp:35-53) and stored as term + 0.0f
 * into a fresh gradient or added. da or db may be NULL; when a and b are one tensor, pass one gradient buffer twice
 * with db_first = 0 (dA is written first). NNH_ERR_SHAPE where the forward's shapes would throw.
 */
int nnh_matmul_backward(const float* g, const float* a, const size_t* a_shape, int a_ndim, const float* b,
                        const size_t* b_shape, int b_ndim, int b_transposed, float* da, int da_first, float* db,
                        int db_first, void* stream);
int nnh_matmul_backward_workspace_size(const size_t* a_shape, int a_ndim, const size_t* b_shape, int b_ndim,
                                       int b_transposed, int want_da, int want_db, size_t* bytes);

/*
 * nn::linear forward (src/autograd/ops.cpp:714-730): y[M x n] = x[M x K] w[n x K]^T, then + bias[n] per
 * column, in one kernel. relu != 0 also applies the ReLU node that follows a Linear in the reference
 * (ops.cpp:775-782) in the same epilogue: y = v > 0 ? v : 0 (bit-identical to linear then relu).
 */
int nnh_linear_forward(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias, int relu,
                       float* y, void* stream);
/*
 * nn::linear, then nn::add(residual, that) (ops.cpp:714-730, 333-336: a transformer block's residual connection) in
 * one kernel: y = residual + (x w^T + bias), element by element the bits of the two ops. No single counterpart in
 * the reference. residual is {M, n}, read before y is written, and may be y itself (not otherwise overlap it).
 */
int nnh_linear_forward_add(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias,
                           const float* residual, float* y, void* stream);
/*
 * nn::linear, then nn::gelu on its output (ops.cpp:714-730, 451-466: a transformer block's fc1 and activation) in one
 * kernel where the product has no depth cut: h {M, n} = x w^T + bias (the GELU's input, which its backward reads),
 * y = gelu(h) and tanh_saved as nnh_gelu_forward leaves them, the bits of the two ops. No single counterpart in the
 * reference. y and tanh_saved overlap neither each other, h, nor the inputs.
 */
int nnh_linear_gelu_forward(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias, float* h,
                            float* y, float* tanh_saved, void* stream);
/*
 * count (1 to 8) nn::linear forwards over one input (ops.cpp:714-730: an attention layer's q, k and v projections):
 * y[i] {M, n[i]} = x w[i]^T + bias[i], the bits of count separate calls, in one launch where the shapes allow (two or
 * three products, each at most 2^20 outputs and 256 deep). No single counterpart in the reference. No output may
 * overlap x, another output, or any layer's weight or bias.
 */
int nnh_linear_forward_multi(const float* x, size_t M, size_t K, int count, const float* const* w, const size_t* n,
                             const float* const* bias, float* const* y, void* stream);

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

/* add_to_grad (src/autograd/ops.cpp:55-82, value.cpp:60-64): a fresh gradient (first) stores src + 0.0f, an
 * existing one adds src, element by element. The first-write rule every backward pass uses; reshape's backward. */
int nnh_add_to_grad(float* dst, const float* src, size_t count, int first, void* stream);

/* nnh_add_to_grad into two gradients of one source in one launch: dst0 by first0's rule, then dst1 by first1's, the
 * backward of an add node whose operands have the output's shape (ops.cpp:333-336; accumulate_grad for a, then b).
 * The two gradients must not overlap each other or src (one node as both operands: two nnh_add_to_grad calls). */
int nnh_add_to_grad2(float* dst0, int first0, float* dst1, int first1, const float* src, size_t count, void* stream);

/* Value::zero_grad over a list of values (Optimizer::zero_grad, src/optim/sgd.cpp:19-21; value.cpp:69-76): n device
 * buffers of counts[i] floats filled with +0, every fill in one launch (64 buffers per launch). The buffers must not
 * overlap one another. */
int nnh_zero_many(float* const* buffers, const size_t* counts, size_t n, void* stream);

/* Tensor::sum(0) of a {rows, inner} tensor (src/tensor.cpp:422-456): s_j = sum of src[a][j] over a in order,
 * from +0. combine 0: dst = s; 1: dst = s + 0.0f (a fresh gradient); 2: dst += s. */
int nnh_tensor_sum0(const float* src, size_t rows, size_t inner, float* dst, int combine, void* stream);

/*
 * nn::attention forward (src/autograd/ops.cpp:1226-1261): q {N, Tq, D}, k and v {N, Tk, D}, `heads` heads of
 * Dh = D / heads columns. probs {N, heads, Tq, Tk} receives the softmax probabilities (kept for the backward
 * pass, as the reference does); out {N, Tq, D}. key_padding_mask {N, Tk} (0 marks a padded key) may be NULL.
 * Shape rules as the reference: NNH_ERR_SHAPE unless heads divides D, Tq, Tk > 0 and (causal => Tq == Tk).
 */
int nnh_attention_forward(const float* q, const float* k, const float* v, size_t N, size_t Tq, size_t Tk, size_t D,
                          size_t heads, const float* key_padding_mask, int causal, float* out, float* probs,
                          void* stream);

/*
 * nn::attention backward (ops.cpp:1263-1295) for upstream gradient g {N, Tq, D} and the forward's probs. Each of
 * dq, dk, dv may be NULL; *_first selects the fresh-gradient rule (overwrite instead of accumulate). When q, k and
 * v are one tensor, pass one gradient buffer three times with dv_first as its freshness and dq_first = dk_first = 0.
 */
int nnh_attention_backward(const float* g, const float* q, const float* k, const float* v, const float* probs,
                           size_t N, size_t Tq, size_t Tk, size_t D, size_t heads, const float* key_padding_mask,
                           int causal, float* dq, int dq_first, float* dk, int dk_first, float* dv, int dv_first,
                           void* stream);

/* nn::scaled_masked_softmax forward (ops.cpp:1298-1322) over x {N, H, Tq, Tk}; x may equal y. */
int nnh_scaled_masked_softmax_forward(const float* x, size_t N, size_t H, size_t Tq, size_t Tk, float scale,
                                      const float* key_padding_mask, int causal, float* y, void* stream);

/* Its backward (ops.cpp:1323-1342): first: dx = masked ? 0 : term + 0.0f; else dx += term where not masked. */
int nnh_scaled_masked_softmax_backward(const float* y, const float* g, size_t N, size_t H, size_t Tq, size_t Tk,
                                       float scale, const float* key_padding_mask, int causal, float* dx, int first,
                                       void* stream);

/*
 * nn::conv2d / nn::conv2d_relu forward (src/autograd/ops.cpp:1345-1410, 1466-1472): x {N, Cin, H, W},
 * w {Cout, Cin, kh, kw}, bias {Cout}, y {N, Cout, Ho, Wo} with Ho = (H + 2 padding - kh) / stride + 1.
 * fuse_relu applies the folded ReLU: v = acc + b; alive = v > 0; y = alive ? v : 0, and alive (optional, one
 * byte per output, laid out like y) receives the flags the backward pass masks with.
 * Shape rules as the reference: NNH_ERR_SHAPE for stride <= 0, padding < 0 or a kernel wider than the padded
 * input.
 */
int nnh_conv2d_forward(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w, size_t Cout,
                       size_t kh, size_t kw, const float* bias, int stride, int padding, int fuse_relu, float* y,
                       unsigned char* alive, void* stream);

/*
 * conv2d_relu (ops.cpp:1396-1416) then maxpool2d(y, pool_kernel, pool_stride) (ops.cpp:1609-1684): y and alive as
 * nnh_conv2d_forward with fuse_relu = 1, pooled and argmax as nnh_maxpool2d_forward on y, the same bits. A
 * network's first layer (stride 1, "same" kh = kw = 2 padding + 1 with padding 1 or 2, W a multiple of 4, H even,
 * Cin (kh + 1) <= 8, a 2 x 2 pool of stride 2, 16-byte aligned x and y, 8-byte aligned pooled and argmax) runs as
 * one kernel that writes all four from registers; other shapes run the two ops in turn. alive and argmax may be
 * NULL. No counterpart in the reference, whose Sequential runs the two modules one after the other.
 */
int nnh_conv2d_relu_maxpool2d_forward(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w,
                                      size_t Cout, size_t kh, size_t kw, const float* bias, int stride, int padding,
                                      size_t pool_kernel, size_t pool_stride, float* y, unsigned char* alive,
                                      float* pooled, unsigned int* argmax, void* stream);

/*
 * Its backward (ops.cpp:1418-1463) for upstream gradient g {N, Cout, Ho, Wo}: g is masked by alive when given
 * (the fused ReLU), db = per-sample lane sums summed over samples in order, dw = per-sample g col^T summed
 * over samples in order, dx = col2im(W^T g). *_first: the gradient is fresh (dx zero-filled first, dw and db
 * stored rather than added). Any of dx, dw, db may be NULL.
 */
int nnh_conv2d_backward(const float* g, const float* x, const float* w, const unsigned char* alive, size_t N,
                        size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride, int padding,
                        float* dx, int dx_first, float* dw, int dw_first, float* db, int db_first, void* stream);

/*
 * Packed forms of the ReLU flags and of the 2 x 2 pool's offsets, for callers whose backward is the flags' only
 * reader (no counterpart in the reference, which keeps one byte per flag and a 32-bit plane offset per window; the
 * byte forms above are unchanged). alive_bits holds one bit per output in y's order: bit o of the flattened
 * {N, Cout, Ho, Wo} index at byte o / 8, bit o % 8 (N Cout Ho Wo / 8 bytes). argmax2 holds each 2 x 2 window's
 * maximum as its 2-bit position in the window (0 row 0 left, 1 row 0 right, 2 row 1 left, 3 row 1 right): window
 * (ph, pw) of plane p at bits 2 (pw % 4) of byte (p (Ho / 2) + ph) ceil(Wo / 8) + pw / 4. Values, gradients and bits
 * are those of the byte forms.
 *
 * nnh_conv2d_packed_supported: 1 when a geometry takes them, both the forward (with_pool: conv2d_relu then a 2 x 2
 * stride-2 maxpool in one pass) and nnh_conv2d_backward_packed (a network's first layer: stride 1, "same" width,
 * Cin kh kw <= 16, Cout <= 32, Ho Wo a multiple of 8, the padded input plane Cin (Ho + kh - 1) (Wo + kw - 1) at most
 * 2048 floats; with the pool H even and W <= 256);
 * pointers must also be aligned as each call states.
 * nnh_conv2d_relu_forward_packed: nnh_conv2d_forward with fuse_relu = 1 and packed flags (x, y 16-byte aligned).
 * nnh_conv2d_relu_maxpool2d_forward_packed: nnh_conv2d_relu_maxpool2d_forward (pool 2, stride 2) with packed flags and
 * offsets (x, y 16-byte, pooled 8-byte aligned).
 * nnh_conv2d_backward_packed: nnh_conv2d_backward with packed flags (g 16-byte aligned).
 * nnh_maxpool2d_backward_packed: nnh_maxpool2d_backward (kernel 2, stride 2) from argmax2 (dx 8-byte aligned).
 */
int nnh_conv2d_packed_supported(size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride,
                                int padding, int with_pool);
int nnh_conv2d_relu_forward_packed(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w,
                                   size_t Cout, size_t kh, size_t kw, const float* bias, int stride, int padding,
                                   float* y, unsigned char* alive_bits, void* stream);
int nnh_conv2d_relu_maxpool2d_forward_packed(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w,
                                             size_t Cout, size_t kh, size_t kw, const float* bias, int stride,
                                             int padding, float* y, unsigned char* alive_bits, float* pooled,
                                             unsigned char* argmax2, void* stream);
int nnh_conv2d_backward_packed(const float* g, const float* x, const float* w, const unsigned char* alive_bits,
                               size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride,
                               int padding, float* dx, int dx_first, float* dw, int dw_first, float* db, int db_first,
                               void* stream);
int nnh_maxpool2d_backward_packed(const float* g, const unsigned char* argmax2, size_t N, size_t C, size_t H, size_t W,
                                  float* dx, int first, void* stream);

/* im2col_sample over a batch (ops.cpp:188-212): col {N, Cin*kh*kw, Ho*Wo}, zeros where a tap is padding. */
int nnh_im2col(const float* x, size_t N, size_t Cin, size_t H, size_t W, size_t kh, size_t kw, int stride, int padding,
               float* col, void* stream);

/* col2im_sample_add over a batch (ops.cpp:224-243): dx {N, Cin, H, W} += the column entries of each element's taps,
 * in the reference's order; first zero-fills dx first. */
int nnh_col2im_add(const float* col, size_t N, size_t Cin, size_t H, size_t W, size_t kh, size_t kw, int stride,
                   int padding, float* dx, int first, void* stream);

/*
 * nn::maxpool2d forward (src/autograd/ops.cpp:1609-1684): x {N, C, H, W}, windows kernel x kernel at stride
 * `stride`, no padding; y {N, C, Ho, Wo} with Ho = (H - kernel) / stride + 1. Each window is scanned row by row from
 * -inf, a value taken only when greater (the first maximum wins; NaN never does; a window with nothing above -inf
 * gives -inf and offset 0). argmax (optional, one uint32 per output) receives the winner's offset inside its
 * (n, c) plane, which the backward pass needs. NNH_ERR_SHAPE where the reference throws TensorShapeError: kernel or
 * stride 0, a kernel larger than the plane, a plane beyond 2^32 elements.
 */
int nnh_maxpool2d_forward(const float* x, size_t N, size_t C, size_t H, size_t W, size_t kernel, size_t stride,
                          float* y, unsigned int* argmax, void* stream);

/* Its backward (ops.cpp:1686-1704): dx {N, C, H, W} (first: zero-filled first, as a fresh gradient) += g at each
 * output's argmax, in output order. */
int nnh_maxpool2d_backward(const float* g, const unsigned int* argmax, size_t N, size_t C, size_t H, size_t W,
                           size_t kernel, size_t stride, float* dx, int first, void* stream);

/*
 * nn::batchnorm forward in training mode (src/autograd/ops.cpp:900-958): x {N, C, S} where S is the product of the
 * axes after the channel axis (S = 1 for BatchNorm1d's {N, C}). Per channel c: mean = (float)(sum over n in order of
 * (double)lane_sum(row (n, c)) / (N*S)), var likewise from lane_sq around the mean, inv_std = 1 / sqrt(var + eps);
 * y = (x - mean) * (weight[c] * inv_std) + bias[c], and with fuse_relu alive = y > 0 (one byte per element, may be
 * NULL) and y clipped at 0 (the fold of BatchNormBase::forward_relu, src/nn/batchnorm.cpp:16-23). mean, var and
 * inv_std receive C floats each (mean and var are the statistics nn-cpp hands its running averages; mean and
 * inv_std are what the backward pass reads); var may be NULL. N*S = 0 gives NaN statistics, as 0/0 does in the
 * reference. Scratch: nnh_batchnorm_workspace_size.
 */
int nnh_batchnorm_forward(const float* x, size_t N, size_t C, size_t S, const float* weight, const float* bias,
                          float eps, int fuse_relu, float* y, unsigned char* alive, float* mean, float* var,
                          float* inv_std, void* stream);

/* Its backward rule (ops.cpp:960-1000). alive: the forward's flags when it folded the ReLU, else NULL. dx (may be
 * NULL) receives k * (M * g' - sum(g') - ((x - mean) * inv_std) * sum(g' (x - mean)) * inv_std) with g' the masked
 * gradient, k = weight * inv_std / M and the two per-channel sums in double over the rows' lane sums; first stores
 * term + 0.0f, else adds. dweight and dbias (may be NULL) have the sums added as the reference's weight.grad() +=
 * does; *_first: the gradient is fresh (0 + sum). */
int nnh_batchnorm_backward(const float* g, const float* x, const unsigned char* alive, const float* weight,
                           const float* mean, const float* inv_std, size_t N, size_t C, size_t S, float* dx,
                           int dx_first, float* dweight, int dweight_first, float* dbias, int dbias_first,
                           void* stream);

/* Scratch of either batchnorm call: two floats per (n, c) row. */
int nnh_batchnorm_workspace_size(size_t N, size_t C, size_t S, size_t* bytes);

/*
 * nn::layernorm forward (ops.cpp:1003-1034) over R rows of D (x {..., D}, gamma and beta {D}): per row the float
 * sum in column order, mean = sum / D, the float sum of squared deviations, inv_std = 1 / sqrt(sq / D + eps),
 * y = (x - mean) * inv_std * gamma + beta. mean and inv_std receive R floats each (the backward pass reads them).
 * D = 0 is refused (NNH_ERR_INVALID: the reference divides by it). No scratch.
 */
int nnh_layernorm_forward(const float* x, size_t R, size_t D, const float* gamma, const float* beta, float eps,
                          float* y, float* mean, float* inv_std, void* stream);

/* Its backward rule (ops.cpp:1035-1077): dx per row (first: term + 0.0f, else added); dgamma and dbeta summed over
 * the rows in order per column and added (first: 0 + sum). Any of the three may be NULL. */
int nnh_layernorm_backward(const float* g, const float* x, const float* gamma, const float* mean, const float* inv_std,
                           size_t R, size_t D, float* dx, int dx_first, float* dgamma, int dgamma_first, float* dbeta,
                           int dbeta_first, void* stream);

/* nn::add (src/autograd/ops.cpp:331-337 forward, src/tensor.cpp:543-545) for a right operand broadcast along the left
 * one's leading axes: y[o][j] = a[o][j] + b[j] over outer x inner (equal shapes: outer 1). y may be a itself. The
 * backward rule is nnh_add_to_grad for a and, for a broadcast b, nnh_tensor_sum0 (sum_to_shape) then the store. */
int nnh_add_forward(const float* a, const float* b, size_t outer, size_t inner, float* y, void* stream);

/* nn::mul (src/autograd/ops.cpp:347-357 forward, src/tensor.cpp:551-553) of two same-shaped tensors: y = a * b. y may
 * be a or b itself. Its backward rule, per operand: d = g * other (the other operand), stored as the product + 0 into a
 * fresh gradient (first), else added (accumulate_grad, ops.cpp:110-117). Dropout's mask multiply uses it
 * (src/nn/dropout.cpp:22-33). */
int nnh_mul_forward(const float* a, const float* b, size_t count, float* y, void* stream);
int nnh_mul_backward(const float* g, const float* other, size_t count, float* d, int first, void* stream);

/* nn::gelu, the tanh form (ops.cpp:451-466): tanh_saved receives tanh(k (x + c x^3)) per element (the reference keeps
 * it for the backward pass), with nn-cpp's own tanh and exp (src/kernels/vmath.cpp:24-105), bit for bit. */
int nnh_gelu_forward(const float* x, size_t count, float* y, float* tanh_saved, void* stream);
/* Its backward rule (ops.cpp:467-480); first: dx is fresh (term + 0.0f), else term is added. */
int nnh_gelu_backward(const float* x, const float* tanh_saved, const float* g, size_t count, float* dx, int first,
                      void* stream);

/* nn::embedding (ops.cpp:1991-2015): y row i = weight row rows[i] for a weight {V, D}. The rows are the ids as int32,
 * validated by the caller (nn-cpp throws TensorShapeError for an id that is negative, fractional or >= V; an id out
 * of range here reads a clamped row). */
int nnh_embedding_forward(const float* weight, size_t V, size_t D, const int* rows, size_t count, float* y,
                          void* stream);
/* nn::embedding, then nn::add(that, addend) with the addend {addend_rows, D} broadcast over the leading rows (row i
 * takes addend row i % addend_rows: a transformer's token embedding plus its positions, ops.cpp:1991-2015 and
 * 333-336) in one kernel, the bits of the two ops. No single counterpart in the reference. addend_rows divides count;
 * y overlaps none of the inputs. */
int nnh_embedding_add_forward(const float* weight, size_t V, size_t D, const int* rows, size_t count,
                              const float* addend, size_t addend_rows, float* y, void* stream);
/* Its backward rule: dweight (first: zero-filled first) += g row i at row rows[i], for i in order. */
int nnh_embedding_backward(const float* g, const int* rows, size_t count, size_t V, size_t D, float* dweight, int first,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NNH_H */
