/*
 * nnh_noalloc.h - an entry point of libnnh that allocates no device memory.
 *
 * No counterpart in the reference: nn::kernels::sgemm (include/nn/kernels/gemm.hpp:57-59) only ever uses host
 * memory. This variant of nnh_sgemm is for callers that cannot allocate: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.
 */
#ifndef NNH_NOALLOC_H
#define NNH_NOALLOC_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * nnh_sgemm (same arguments, same bits), with its only scratch, the depth-cut partial sums, in a static device
 * array of nnh_sgemm_noalloc_max_workspace() bytes (16 MiB) that each GPU holds until the process ends. It calls
 * no hipMalloc, hipFree or allocating library routine. Partial sums are written only by products cut into more
 * than 16 pieces (nn-cpp's rule with k > 2048: m n k / 128 floats, rounded up to whole pieces); one whose partials
 * exceed the array returns NNH_ERR_INVALID without launching anything.
 * All calls on one GPU share that GPU's array: calls on one stream run in order, but calls that overlap on one GPU
 * (different streams, unordered) race on it.
 */
int nnh_sgemm_noalloc(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                      const float* b, size_t ldb, float* c, size_t ldc, int accumulate, void* stream);

/* Size in bytes of the static scratch array nnh_sgemm_noalloc uses. */
size_t nnh_sgemm_noalloc_max_workspace(void);

#ifdef __cplusplus
}
#endif

#endif /* NNH_NOALLOC_H */
