// Plain-C launch descriptors shared by the C++ host planner and the HIP
// kernels. The host proves every address of a launch in bounds before it
// fills one of these; the device code never sees the Kernel IR itself.
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/// Element types a device buffer may hold (KernelBuffer::dtype subset,
/// compiler/include/mlk/type/domain.h:53-60).
enum mlkd_dtype { MLKD_F32 = 0, MLKD_F16 = 1, MLKD_F64 = 2 };

/// Runtime scalar parameters of a chain (ScalarParam operands,
/// kernel_ir.h:58-70); indices past the bound table read 0.0 like the
/// reference evaluator (kernel_buffers.cpp:114-117).
enum { MLKD_MAX_SCALARS = 8 };
typedef struct mlkd_scalars {
    double v[MLKD_MAX_SCALARS];
} mlkd_scalars;

/// Row softmax / row sum: Y[r, :] = f(X[r, :]) over rows x cols, row strides
/// in elements.
typedef struct mlkd_softmax {
    const void* x;
    void* y;
    int32_t x_dtype, y_dtype;
    int64_t rows, cols;
    int64_t x_row_stride, y_row_stride;
    int32_t variant;     /* launch form; -1: the process default */
    int32_t pad;
} mlkd_softmax;

/// C[M,N] (+)= A[M,K] * B[K,N], row-major, leading dims in elements.
typedef struct mlkd_gemm {
    const void* a;
    const void* b;
    void* c;
    int32_t a_dtype, b_dtype, c_dtype;
    int32_t accumulate;   /* 1: C += A*B (Call form); 0: C = A*B */
    int64_t m, n, k;
    int64_t lda, ldb, ldc;
    int32_t variant;      /* launch form; -1: the process default */
    /* 1: skip the products of A[i,p] == 0, the reference's gemmRowBlock
       (kernel_buffers.cpp:422), with C[i,j] = C_in + sum over p ascending.
       With `accumulate`, the MFMA forms run it: a wave whose accumulators
       met an infinity or a NaN (only there can the skip change C) recomputes
       its block exactly. Otherwise the general kernel runs everything. */
    int32_t skip_zero_a;
    int32_t pad_;
    /* Device workspace for shapes the MFMA forms do not tile
       (mlkd_gemm_pad_bytes): the operands are copied into zero-padded
       blocks there, the MFMA form runs on them and C is copied back. NULL
       (or too small) keeps such shapes on the general kernel. */
    void* work;
    int64_t work_bytes;
} mlkd_gemm;

/// S[b*seq + i, j] = softmax_j((Q[b,i,:] . K[b,j,:]) / div + bias[j]).
typedef struct mlkd_score_softmax {
    const void* q;
    const void* k;
    const void* bias;
    void* s;
    int32_t qk_dtype, bias_dtype, s_dtype;
    int32_t variant;      /* launch form; -1: the process default */
    int64_t batch, seq, dim;
    double div;
    /* Device scratch for the two-pass form's per-tile row statistics
       (mlkd_score_scratch_bytes); may be NULL, which selects another form. */
    void* scratch;
    int64_t scratch_bytes;
    /* Workspace for a sequence length off the two-pass form's 256-row blocks
       (mlkd_score_pad_bytes): Q, K and the bias are copied into zero-padded
       blocks (padded keys get a -inf bias), the two passes run there and S
       is copied back. NULL (or too small) keeps such shapes on the general
       kernels. */
    void* work;
    int64_t work_bytes;
} mlkd_score_softmax;

#ifdef __cplusplus
}
#endif
