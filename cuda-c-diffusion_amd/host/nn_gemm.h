/* nn_gemm.h -- row-major fp32 GEMMs on rocBLAS for the modules that wrap a
 * GEMM around the fused kernels (mp_linear, conv2d).  The GEMM itself is
 * outside the fused-kernel path; these mirror the row-major helpers of the
 * reference (src/gemm.h:10-38).  rocBLAS is column-major, so a row-major
 * [r, c] matrix is read as its transpose with leading dimension c.
 */
#ifndef NN_GEMM_H
#define NN_GEMM_H

#include "nn_modules.h"

/* Y[batch,out] = alpha * X[batch,in] @ W[in,out] */
static inline void nn_gemm_forward(rocblas_handle h, float alpha, const float* X, const float* W,
    float* Y, int batch, int in, int out)
{
    const float beta = 0.0f;
    NN_BLAS_CHECK(rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_none, out, batch, in,
        &alpha, W, out, X, in, &beta, Y, out));
}

/* gW[in,out] = alpha * X[batch,in]^T @ dZ[batch,out] */
static inline void nn_gemm_dW(rocblas_handle h, float alpha, const float* X, const float* dZ,
    float* gW, int batch, int in, int out)
{
    const float beta = 0.0f;
    NN_BLAS_CHECK(rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_transpose, out, in,
        batch, &alpha, dZ, out, X, in, &beta, gW, out));
}

/* dX[batch,in] = alpha * dZ[batch,out] @ W[in,out]^T */
static inline void nn_gemm_dX(rocblas_handle h, float alpha, const float* W, const float* dZ,
    float* dX, int batch, int in, int out)
{
    const float beta = 0.0f;
    NN_BLAS_CHECK(rocblas_sgemm(h, rocblas_operation_transpose, rocblas_operation_none, in, batch,
        out, &alpha, W, out, dZ, out, &beta, dX, in));
}

#endif /* NN_GEMM_H */
