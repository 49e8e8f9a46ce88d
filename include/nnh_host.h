/*
 * nnh_host.h - C entry of the drop-in nn::kernels::sgemm (lib/libnn_gemm_hip.so).
 *
 * libnn_gemm_hip.so defines nn::kernels::sgemm, sgemm_portable, sgemm_unpacked and sgemm_uses_avx2 with the exact
 * signatures of nn-cpp's include/nn/kernels/gemm.hpp:57-94, over HOST pointers, so it replaces src/kernels/gemm.cpp
 * at link time. Each call stages its operands to the GPU, runs nnh_sgemm and copies C back; the result is
 * bit-identical to nn-cpp's AVX2 build. This C function is the same operation for callers without C++.
 */
#ifndef NNH_HOST_H
#define NNH_HOST_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* nn::kernels::sgemm (include/nn/kernels/gemm.hpp:57-59) on host memory. Returns NNH_OK or NNH_ERR_HIP. */
int nnh_sgemm_host(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b,
                   size_t ldb, float* c, size_t ldc, int accumulate);

/* Number of products the drop-in has run in this process. */
unsigned long long nnh_sgemm_host_calls(void);

#ifdef __cplusplus
}
#endif

#endif /* NNH_HOST_H */
