// Config-5 class: S[b*seq + i, :] = softmax((Q[b,i,:] . K[b,:,:]^T) / div +
// bias), the composition of Call(MatMul) (kernel_buffers.cpp:406-432), the
// broadcast elementwise chain Add(Div(S, c), bias[j]) (poly.synth.cpp:
// 231-353) and the stable softmax (kernel_buffers.cpp:290-340).
//
// The output write (4 * batch * seq^2 bytes) bounds the class; the scores are
// a GEMM with K = dim on v_mfma_f32_32x32x16_f16. Forms, best first:
//   * two-pass, query-stationary (dim 128, seq % 256 == 0, seq <= 8192): a
//     statistics pass and a recompute-and-write pass (scoreStatsQ /
//     scoreStoreQ), rows' partial statistics in artifact scratch;
//   * two-pass on 256 x 256 blocks (any seq % 256 == 0);
//   * fused single pass holding a 32-row block in registers (seq <= 2048);
//   * scores, then the softmax kernel in place over S (any shape, f16);
//   * a scalar f64 path for other dtypes.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "mlk_device_math.h"
#include "runtime_abi.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void scoresF16(const _Float16* __restrict__ Q,
                                                 const _Float16* __restrict__ K,
                                                 const float* __restrict__ bias,
                                                 float* __restrict__ S, int seq, int dim,
                                                 float div) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tilesJ = seq / 128;
    const int tilesI = seq / 64;
    const int64_t b = blockIdx.x / (tilesI * tilesJ);
    const int rem = blockIdx.x % (tilesI * tilesJ);
    const int i0 = (rem / tilesJ) * 64 + (wave >> 1) * 32;
    const int j0 = (rem % tilesJ) * 128 + (wave & 1) * 64;
    const _Float16* q = Q + (b * seq + i0 + (lane & 31)) * dim + (lane >> 5) * 8;
    const _Float16* k0 = K + (b * seq + j0 + (lane & 31)) * dim + (lane >> 5) * 8;
    const _Float16* k1 = k0 + static_cast<int64_t>(32) * dim;
    f32x16 acc0, acc1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        acc0[r] = 0.0f;
        acc1[r] = 0.0f;
    }
    for (int kk = 0; kk < dim; kk += 16) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(q + kk);
        const f16x8 x0 = *reinterpret_cast<const f16x8*>(k0 + kk);
        const f16x8 x1 = *reinterpret_cast<const f16x8*>(k1 + kk);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, x0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, x1, acc1, 0, 0, 0);
    }
    const int col = lane & 31;
    const float bj0 = bias[j0 + col];
    const float bj1 = bias[j0 + 32 + col];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t row = b * seq + i0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        float* dst = S + row * seq + j0 + col;
        dst[0] = acc0[r] / div + bj0;
        dst[32] = acc1[r] / div + bj1;
    }
}

/// Fused single pass (seq <= 2048, seq % 128 == 0, dim % 16 == 0,
/// dim <= 256): a workgroup owns 32 query rows of one batch and all seq key
/// columns. Wave w computes the 32 x (seq/4) score block of columns
/// [w*seq/4, (w+1)*seq/4) with v_mfma_f32_32x32x16_f16, keeping it in
/// accumulators (seq/128 tiles of 32x32, at most 16 tiles = 256 AGPRs).
/// Scale and bias are applied in registers, the row max and row sum are
/// reduced across the 32 lanes of a half-wave (shuffles) and across the 4
/// waves (LDS), and each normalized score is written to HBM exactly once:
/// the kernel's HBM traffic is Q, K (L2-resident per batch) and one write
/// of S.
template <int NT>
__global__ __launch_bounds__(256) void scoreSoftmaxFused(const _Float16* __restrict__ Q,
                                                         const _Float16* __restrict__ K,
                                                         const float* __restrict__ bias,
                                                         float* __restrict__ S, int seq, int dim,
                                                         float div) {
    __shared__ float redMax[4][32];
    __shared__ float redSum[4][32];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rowsPerBatch = seq / 32;
    const int64_t b = blockIdx.x / rowsPerBatch;
    const int i0 = (blockIdx.x % rowsPerBatch) * 32;
    const int j0 = wave * (NT * 32);
    const int l32 = lane & 31;
    const int half = lane >> 5;
    const _Float16* q = Q + (b * seq + i0 + l32) * dim + half * 8;
    const _Float16* kbase = K + (b * seq + j0 + l32) * dim + half * 8;
    f32x16 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
    }
    for (int kk = 0; kk < dim; kk += 16) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(q + kk);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const f16x8 x = *reinterpret_cast<const f16x8*>(kbase + static_cast<int64_t>(t) * 32 * dim + kk);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, x, acc[t], 0, 0, 0);
        }
    }
    // Scale + bias; per-lane row maxima (register r holds row
    // 8*(r/4) + 4*half + r%4 of the tile, column l32).
    float rmax[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) rmax[r] = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float bj = bias[j0 + t * 32 + l32];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float v = acc[t][r] / div + bj;
            acc[t][r] = v;
            rmax[r] = fmaxf(rmax[r], v);
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) rmax[r] = fmaxf(rmax[r], __shfl_xor(rmax[r], off, 64));
    }
    if (l32 == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) redMax[wave][8 * (r >> 2) + 4 * half + (r & 3)] = rmax[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * half + (r & 3);
        rmax[r] = fmaxf(fmaxf(redMax[0][row], redMax[1][row]), fmaxf(redMax[2][row], redMax[3][row]));
    }
    float rsum[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) rsum[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float e = __expf(acc[t][r] - rmax[r]);
            acc[t][r] = e;
            rsum[r] += e;
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) rsum[r] += __shfl_xor(rsum[r], off, 64);
    }
    if (l32 == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) redSum[wave][8 * (r >> 2) + 4 * half + (r & 3)] = rsum[r];
    }
    __syncthreads();
    float inv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * half + (r & 3);
        const float sum = (redSum[0][row] + redSum[1][row]) + (redSum[2][row] + redSum[3][row]);
        inv[r] = sum != 0.0f ? 1.0f / sum : 0.0f;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float* dst = S + (b * seq + i0) * static_cast<int64_t>(seq) + j0 + t * 32 + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r >> 2) + 4 * half + (r & 3);
            __builtin_nontemporal_store(acc[t][r] * inv[r], dst + static_cast<int64_t>(row) * seq);
        }
    }
}

/// Fused single pass, second form (dim = 16*KS with KS in {4, 8}, seq =
/// 32*NT*WAVES): WAVES waves per workgroup split the seq columns, each wave
/// keeps NT 32x32 score tiles in accumulators. The dim loop is unrolled at
/// compile time; Q fragments load once, and tile t+1's K fragments are
/// loaded while tile t's MFMAs run. With WAVES = 8 and NT = 8 a wave needs
/// 128 AGPRs, so two waves share each SIMD and one wave's stores overlap
/// another's MFMAs. Workgroups of one batch are placed on one XCD
/// (logical id = (id % 8) * (total / 8) + id / 8), so each batch's K is
/// fetched into a single L2.
template <int WAVES, int NT, int KS>
__global__ __launch_bounds__(WAVES * 64) void scoreSoftmaxFusedT(const _Float16* __restrict__ Q,
                                                                const _Float16* __restrict__ K,
                                                                const float* __restrict__ bias,
                                                                float* __restrict__ S, int seq,
                                                                float div) {
    constexpr int kDim = KS * 16;
    __shared__ float redMax[WAVES][32];
    __shared__ float redSum[WAVES][32];
    // Output staging: 16 rows x (NT*32 + 4) floats per wave, so each global
    // store writes one contiguous row span of the wave (NT*128 bytes).
    constexpr int kStageW = NT * 32 + 4;
    __shared__ __align__(16) float stage[WAVES][16 * kStageW];
    const float rdiv = 1.0f / div;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rowsPerBatch = seq / 32;
    const int total = static_cast<int>(gridDim.x);
    int id = static_cast<int>(blockIdx.x);
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    const int64_t b = id / rowsPerBatch;
    const int i0 = (id % rowsPerBatch) * 32;
    const int j0 = wave * (NT * 32);
    const int l32 = lane & 31;
    const int half = lane >> 5;
    const _Float16* q = Q + (b * seq + i0 + l32) * kDim + half * 8;
    const _Float16* kbase = K + (b * seq + j0 + l32) * kDim + half * 8;
    f16x8 a[KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) a[k] = *reinterpret_cast<const f16x8*>(q + k * 16);
    f16x8 xb[2][KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) xb[0][k] = *reinterpret_cast<const f16x8*>(kbase + k * 16);
    f32x16 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (t + 1 < NT) {
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                xb[(t + 1) & 1][k] =
                    *reinterpret_cast<const f16x8*>(kbase + static_cast<int64_t>(t + 1) * 32 * kDim + k * 16);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[k], xb[t & 1][k], acc[t], 0, 0, 0);
    }
    float rmax[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) rmax[r] = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float bj = bias[j0 + t * 32 + l32];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float v = acc[t][r] * rdiv + bj;
            acc[t][r] = v;
            rmax[r] = fmaxf(rmax[r], v);
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) rmax[r] = fmaxf(rmax[r], __shfl_xor(rmax[r], off, 64));
    }
    if (l32 == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) redMax[wave][8 * (r >> 2) + 4 * half + (r & 3)] = rmax[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * half + (r & 3);
        float m = redMax[0][row];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) m = fmaxf(m, redMax[w][row]);
        rmax[r] = m;
    }
    float rsum[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) rsum[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float e = __expf(acc[t][r] - rmax[r]);
            acc[t][r] = e;
            rsum[r] += e;
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) rsum[r] += __shfl_xor(rsum[r], off, 64);
    }
    if (l32 == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) redSum[wave][8 * (r >> 2) + 4 * half + (r & 3)] = rsum[r];
    }
    __syncthreads();
    float inv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * half + (r & 3);
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) sum += redSum[w][row];
        inv[r] = sum != 0.0f ? 1.0f / sum : 0.0f;
    }
    float* stg = stage[wave];
    float* rowBase = S + (b * seq + i0) * static_cast<int64_t>(seq) + j0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        // Registers 8h..8h+7 hold rows 16h..16h+15 of every tile.
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const int r = 8 * h + rr;
                const int rowLocal = 8 * (rr >> 2) + 4 * half + (rr & 3);
                stg[rowLocal * kStageW + t * 32 + l32] = acc[t][r] * inv[r];
            }
        }
        __syncthreads();
        // Each row of the wave's span is NT*32 floats = NT*8 float4.
#pragma unroll
        for (int q = lane; q < 16 * NT * 8; q += 64) {
            const int rowLocal = q / (NT * 8);
            const int c4 = q - rowLocal * (NT * 8);
            const f32x4 v = *reinterpret_cast<const f32x4*>(stg + rowLocal * kStageW + c4 * 4);
            __builtin_nontemporal_store(
                v, reinterpret_cast<f32x4*>(rowBase + static_cast<int64_t>(16 * h + rowLocal) * seq + c4 * 4));
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------ two pass ----
// Two-pass recompute form (dim 128, seq a multiple of 256): the score matrix
// is a GEMM with K = 128, so recomputing it costs less than holding a row
// block in registers while it is written. Both passes tile D in ROWS x COLS
// blocks; a workgroup has (ROWS/64) x (COLS/128) waves, each computing a
// 64 x 128 sub-block as 2 x 4 v_mfma_f32_32x32x16_f16 tiles from operand
// panels staged in LDS (16-byte row padding: conflict-free 16-byte reads).
// KST is the head-dim width staged per step: 128 stages each panel once,
// 64 stages two halves through one buffer with the second half's global
// loads in flight during the first half's MFMAs.
//   Pass 1 (scoreStats2) computes D = K Q^T (keys x queries), so a query's
//   scores lie in one lane's accumulators: it reduces max and
//   sum(exp(v - max)) over 64 keys in registers (one exchange with the lane
//   32 away), combines the key waves through LDS and writes the pair for its
//   ROWS-key block to scratch[row][key block].
//   Pass 2 (scoreStore2) combines a row's partials, computes D = Q K^T
//   (queries x keys) and writes exp(v - max) / sum to S, each 32-lane
//   half-wave one 128-byte line per store (plain stores, or nontemporal).
// Both evaluate v = acc * (1/div) + bias[j] with the same operations on the
// same MFMA results. Workgroups of one batch run on one XCD, whose L2 then
// holds that batch's Q and K.
constexpr int kD2 = 128;                 // head dim
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

/// Threads of a workgroup of (rows/64) x (cols/128) waves.
constexpr int threads2(int rows, int cols) { return (rows / 64) * (cols / 128) * 64; }

template <int ROWS, int COLS, int KST>
struct Shape2 {
    static constexpr int kWaves = (ROWS / 64) * (COLS / 128);
    static constexpr int kThreads = kWaves * 64;
    static constexpr int kRow = KST + 8;                       // halves per LDS row
    static constexpr int kChunksRow = KST / 8;                 // 16-byte chunks per staged row
    static constexpr int kChunks = (ROWS + COLS) * kChunksRow;
    static constexpr int kPer = kChunks / kThreads;            // chunks per thread per stage
    static constexpr size_t kLds = static_cast<size_t>(ROWS + COLS) * kRow * sizeof(_Float16);
    static_assert(kChunks % kThreads == 0, "stage must split evenly over the threads");
};

/// Global -> registers for one head-dim stage of the two panels: ROWS rows of
/// `m`, then COLS rows of `n`.
template <class SH, int ROWS>
__device__ __forceinline__ void loadStage2(const _Float16* __restrict__ m, const _Float16* __restrict__ n,
                                           int stage, int tid, u32x4v (&v)[SH::kPer]) {
#pragma unroll
    for (int j = 0; j < SH::kPer; ++j) {
        const int c = j * SH::kThreads + tid;
        const int r = c / SH::kChunksRow;
        const int ch = c % SH::kChunksRow;
        const _Float16* src = r < ROWS ? m + r * kD2 : n + (r - ROWS) * kD2;
        v[j] = *reinterpret_cast<const u32x4v*>(src + stage * SH::kChunksRow * 8 + ch * 8);
    }
}

template <class SH>
__device__ __forceinline__ void storeStage2(_Float16* lds, int tid, const u32x4v (&v)[SH::kPer]) {
#pragma unroll
    for (int j = 0; j < SH::kPer; ++j) {
        const int c = j * SH::kThreads + tid;
        *reinterpret_cast<u32x4v*>(lds + (c / SH::kChunksRow) * SH::kRow + (c % SH::kChunksRow) * 8) = v[j];
    }
}

/// acc[2][4] += the wave's 64 x 128 sub-block over one staged head-dim range.
template <class SH, int ROWS, int KST>
__device__ __forceinline__ void mfmaStage2(const _Float16* lds, int wm, int wn, int l32, int hl,
                                           f32x16 (&acc)[2][4]) {
    const _Float16* pm = lds;
    const _Float16* pn = lds + ROWS * SH::kRow;
#pragma unroll
    for (int ks = 0; ks < KST / 16; ++ks) {
        f16x8 a[2], x[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a[i] = *reinterpret_cast<const f16x8*>(pm + (wm * 64 + i * 32 + l32) * SH::kRow + ks * 16 + hl * 8);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[j] = *reinterpret_cast<const f16x8*>(pn + (wn * 128 + j * 32 + l32) * SH::kRow + ks * 16 + hl * 8);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], x[j], acc[i][j], 0, 0, 0);
            }
        }
    }
}

/// The block's ROWS x COLS products over K = 128 (m: ROWS rows, n: COLS rows).
template <int ROWS, int COLS, int KST>
__device__ __forceinline__ void blockProduct2(const _Float16* __restrict__ m, const _Float16* __restrict__ n,
                                              _Float16* lds, int tid, f32x16 (&acc)[2][4]) {
    using SH = Shape2<ROWS, COLS, KST>;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / (COLS / 128), wn = wave % (COLS / 128), l32 = lane & 31, hl = lane >> 5;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
    }
    u32x4v v[SH::kPer];
    loadStage2<SH, ROWS>(m, n, 0, tid, v);
    storeStage2<SH>(lds, tid, v);
    __syncthreads();
    if constexpr (KST == kD2) {
        mfmaStage2<SH, ROWS, KST>(lds, wm, wn, l32, hl, acc);
    } else {
#pragma unroll
        for (int st = 1; st < kD2 / KST; ++st) {
            loadStage2<SH, ROWS>(m, n, st, tid, v);   // in flight during the previous stage's MFMAs
            mfmaStage2<SH, ROWS, KST>(lds, wm, wn, l32, hl, acc);
            __syncthreads();
            storeStage2<SH>(lds, tid, v);
            __syncthreads();
        }
        mfmaStage2<SH, ROWS, KST>(lds, wm, wn, l32, hl, acc);
    }
}

/// Block coordinates: batch, block row and block column. A batch's blocks
/// are contiguous within one XCD's share of the grid.
__device__ __forceinline__ void blockOf2(int rowsB, int colsB, int64_t& b, int& tr, int& tc) {
    const int total = static_cast<int>(gridDim.x);
    int id = static_cast<int>(blockIdx.x);
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    b = id / (rowsB * colsB);
    const int rem = id % (rowsB * colsB);
    tr = rem / colsB;
    tc = rem % colsB;
}

template <int ROWS, int COLS, int KST>
__global__ __launch_bounds__(threads2(ROWS, COLS), 512 / threads2(ROWS, COLS))
void scoreStats2(const _Float16* __restrict__ Q, const _Float16* __restrict__ K, const float* __restrict__ bias,
                 float2* __restrict__ part, int seq, float rdiv) {
    constexpr int WN = COLS / 128;
    constexpr int WM = ROWS / 64;
    extern __shared__ __align__(16) _Float16 lds2[];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN, l32 = lane & 31, hl = lane >> 5;
    const int nKB = seq / ROWS;          // key blocks (rows of D here)
    int64_t b;
    int tk, tq;
    blockOf2(nKB, seq / COLS, b, tk, tq);
    float bk[2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) bk[i][r] = bias[tk * ROWS + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * hl + (r & 3)];
    }
    f32x16 acc[2][4];
    blockProduct2<ROWS, COLS, KST>(K + (b * seq + static_cast<int64_t>(tk) * ROWS) * kD2,
                                   Q + (b * seq + static_cast<int64_t>(tq) * COLS) * kD2, lds2, tid, acc);
    float pm[4], pl[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float v = acc[i][j][r] * rdiv + bk[i][r];
                acc[i][j][r] = v;
                mx = fmaxf(mx, v);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        float l = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) l += __expf(acc[i][j][r] - mx);
        }
        pm[j] = mx;
        pl[j] = l + __shfl_xor(l, 32, 64);
    }
    // Combine the key waves of each query through LDS: [WM][COLS] max, then sum.
    __syncthreads();
    float* red = reinterpret_cast<float*>(lds2);
    if (hl == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            red[wm * COLS + wn * 128 + j * 32 + l32] = pm[j];
            red[(WM + wm) * COLS + wn * 128 + j * 32 + l32] = pl[j];
        }
    }
    __syncthreads();
    for (int q = tid; q < COLS; q += Shape2<ROWS, COLS, KST>::kThreads) {
        float mx = red[q];
#pragma unroll
        for (int w = 1; w < WM; ++w) mx = fmaxf(mx, red[w * COLS + q]);
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < WM; ++w) l += red[(WM + w) * COLS + q] * __expf(red[w * COLS + q] - mx);
        part[(b * seq + static_cast<int64_t>(tq) * COLS + q) * nKB + tk] = make_float2(mx, l);
    }
}

template <int ROWS, int COLS, int KST, bool NT>
__global__ __launch_bounds__(threads2(ROWS, COLS), 512 / threads2(ROWS, COLS))
void scoreStore2(const _Float16* __restrict__ Q, const _Float16* __restrict__ K, const float* __restrict__ bias,
                 const float2* __restrict__ part, float* __restrict__ S, int seq, int nKB, float rdiv) {
    constexpr int WN = COLS / 128;
    extern __shared__ __align__(16) _Float16 lds2[];
    __shared__ float rowMax[ROWS];
    __shared__ float rowInv[ROWS];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN, l32 = lane & 31, hl = lane >> 5;
    int64_t b;
    int tq, tk;
    blockOf2(seq / ROWS, seq / COLS, b, tq, tk);
    const int64_t row0 = b * seq + static_cast<int64_t>(tq) * ROWS;
    for (int rr = tid; rr < ROWS; rr += Shape2<ROWS, COLS, KST>::kThreads) {
        const float2* pr = part + (row0 + rr) * nKB;
        float mx = -INFINITY;
        for (int p = 0; p < nKB; ++p) mx = fmaxf(mx, pr[p].x);
        float l = 0.0f;
        for (int p = 0; p < nKB; ++p) l += pr[p].y * __expf(pr[p].x - mx);
        rowMax[rr] = mx;
        rowInv[rr] = l != 0.0f ? 1.0f / l : 0.0f;
    }
    float bj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bj[j] = bias[tk * COLS + wn * 128 + j * 32 + l32];
    f32x16 acc[2][4];
    blockProduct2<ROWS, COLS, KST>(Q + row0 * kD2, K + (b * seq + static_cast<int64_t>(tk) * COLS) * kD2, lds2, tid,
                                   acc);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int rl = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
            const float mx = rowMax[rl];
            const float inv = rowInv[rl];
            float* dst = S + (row0 + rl) * static_cast<int64_t>(seq) + tk * COLS + wn * 128 + l32;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float o = __expf(acc[i][j][r] * rdiv + bj[j] - mx) * inv;
                if constexpr (NT) {
                    __builtin_nontemporal_store(o, dst + j * 32);
                } else {
                    dst[j * 32] = o;
                }
            }
        }
    }
}

// Query-stationary form of the two passes (dim 128, seq a multiple of 256).
// A wave owns 32 query rows and holds their Q fragments in registers for the
// whole kernel; a workgroup of 4 waves (128 rows) streams one half of the
// batch's keys through LDS in 128-key panels, double buffered, the next
// panel's global loads in flight during the current panel's MFMAs. 73 KiB
// of LDS and <= 256 registers per lane let two workgroups share a CU.
//   Pass 1 (scoreStatsQ) computes D = K Q^T per panel, so each lane holds 64
//   of its query's scores per panel and keeps a running max and
//   sum(exp(v - max)) in two registers; the lane 32 away holds the other
//   keys of the same query, and the pair is combined once at the end into
//   scratch[row][key half].
//   Pass 2 (scoreStoreQ) computes D = Q K^T per panel and writes
//   exp(v - max) / sum for the panel at once: each 32-lane half-wave stores
//   one 128-byte line, while the other workgroup on the CU computes.
// Both passes work in base 2 with log2(e) folded into 1/div and the bias, so
// a score costs one fused multiply-add and one v_exp_f32: the passes are
// bound by VALU work (67M exponentials each), not by the MFMAs.
constexpr int kPanelQ = 128;                   // keys per streamed panel
constexpr float kLog2e = 1.44269504088896340736f;
constexpr int kRowQ = kD2 + 8;                 // halves per LDS panel row
constexpr int kPanelHalvesQ = kPanelQ * kRowQ;
constexpr size_t kLdsStoreQ = 2 * kPanelHalvesQ * sizeof(_Float16);  // pass 1 adds seq/2 floats of bias
constexpr int64_t kMaxSeqQ = 8192;             // pass 1's LDS stays <= 86 KiB

/// 256 threads: global -> registers for one 128-key panel (8 chunks each).
__device__ __forceinline__ void loadPanelQ(const _Float16* __restrict__ k, int tid, u32x4v (&v)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = j * 256 + tid;
        v[j] = *reinterpret_cast<const u32x4v*>(k + (c >> 4) * kD2 + (c & 15) * 8);
    }
}

__device__ __forceinline__ void storePanelQ(_Float16* dst, int tid, const u32x4v (&v)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = j * 256 + tid;
        *reinterpret_cast<u32x4v*>(dst + (c >> 4) * kRowQ + (c & 15) * 8) = v[j];
    }
}

/// Workgroup coordinates: batch, 128-row block, key half. A batch's
/// workgroups are contiguous within one XCD's share of the grid.
__device__ __forceinline__ void blockOfQ(int rowBlocks, int64_t& b, int& rb, int& kh) {
    const int total = static_cast<int>(gridDim.x);
    int id = static_cast<int>(blockIdx.x);
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    b = id / (rowBlocks * 2);
    const int rem = id % (rowBlocks * 2);
    rb = rem / 2;
    kh = rem % 2;
}

/// Pass-1 statistics of this wave's 32 queries of row block (b, rb) over
/// keys [k0, k0 + keys): D = K Q^T per 128-key panel, so each lane keeps a
/// running max and sum(exp2(v - max)) of its query; the lane 32 away holds
/// the other keys of the same query and the pair is combined at the end.
/// Returns (max, sum) of query row `qrow` in base 2 (both half-waves agree).
__device__ __forceinline__ float2 statsRangeQ(const _Float16* __restrict__ Q, const _Float16* __restrict__ K,
                                              const float* __restrict__ bias, int seq, float c2, int64_t b,
                                              int rb, int k0, int keys, _Float16* ldsQ, int64_t& qrow) {
    float* lbias = reinterpret_cast<float*>(ldsQ + 2 * kPanelHalvesQ);  // this key range's bias
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, l32 = lane & 31, hl = lane >> 5;
    const int np = keys / kPanelQ;
    qrow = b * seq + static_cast<int64_t>(rb) * 128 + wave * 32 + l32;
    f16x8 xq[8];                                  // B operand: this lane's query, 8 x 16 head dims
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) xq[ks] = *reinterpret_cast<const f16x8*>(Q + qrow * kD2 + ks * 16 + hl * 8);
    for (int i = tid; i < keys; i += 256) lbias[i] = bias[k0 + i] * kLog2e;
    const _Float16* kb = K + (b * seq + k0) * kD2;
    u32x4v v[8];
    loadPanelQ(kb, tid, v);
    storePanelQ(ldsQ, tid, v);
    __syncthreads();
    float m = -INFINITY, l = 0.0f;
    for (int p = 0; p < np; ++p) {
        if (p + 1 < np) loadPanelQ(kb + static_cast<int64_t>(p + 1) * kPanelQ * kD2, tid, v);
        const _Float16* pk = ldsQ + (p & 1) * kPanelHalvesQ;
        f32x16 acc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(pk + (i * 32 + l32) * kRowQ + ks * 16 + hl * 8);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, xq[ks], acc[i], 0, 0, 0);
            }
        }
        // acc[i][r]: key p*128 + i*32 + 8*(r/4) + 4*hl + r%4 of this lane's query.
        float mb = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 bb = *reinterpret_cast<const f32x4*>(lbias + p * kPanelQ + i * 32 + 8 * g + 4 * hl);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float x = __builtin_fmaf(acc[i][4 * g + q], c2, bb[q]);
                    acc[i][4 * g + q] = x;
                    mb = fmaxf(mb, x);
                }
            }
        }
        const float mn = fmaxf(m, mb);
        float sb = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sb += __builtin_amdgcn_exp2f(acc[i][r] - mn);
        }
        l = l * __builtin_amdgcn_exp2f(m - mn) + sb;
        m = mn;
        if (p + 1 < np) storePanelQ(ldsQ + ((p + 1) & 1) * kPanelHalvesQ, tid, v);
        __syncthreads();
    }
    const float mo = __shfl_xor(m, 32, 64);
    const float lo = __shfl_xor(l, 32, 64);
    const float mx = fmaxf(m, mo);
    const float lt = l * __builtin_amdgcn_exp2f(m - mx) + lo * __builtin_amdgcn_exp2f(mo - mx);
    return make_float2(mx, lt);
}

/// Row statistics of the 16 rows this lane's pass-2 accumulators hold,
/// merged from NP key-range partials part[row * NP + i] (base 2).
template <int NP>
__device__ __forceinline__ void mergeStatsQ(const float2* __restrict__ part, int64_t r0, float (&rmx)[16],
                                            float (&rinv)[16]) {
    const int hl = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float2* pr = part + (r0 + 8 * (r >> 2) + 4 * hl + (r & 3)) * NP;
        float2 pp[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) pp[i] = pr[i];
        float mx = pp[0].x;
#pragma unroll
        for (int i = 1; i < NP; ++i) mx = fmaxf(mx, pp[i].x);
        float lt = 0.0f;
#pragma unroll
        for (int i = 0; i < NP; ++i) lt += pp[i].y * __builtin_amdgcn_exp2f(pp[i].x - mx);
        rmx[r] = mx;
        rinv[r] = lt != 0.0f ? 1.0f / lt : 0.0f;
    }
}

/// Pass 2 over keys [k0, k0 + keys) of this wave's 32 rows r0..r0+31 of
/// batch b: D = Q K^T per panel, written as exp2(v - max) / sum at once;
/// each 32-lane half-wave stores one 128-byte line.
__device__ __forceinline__ void storeRangeQ(const _Float16* __restrict__ Q, const _Float16* __restrict__ K,
                                            const float* __restrict__ bias, float* __restrict__ S, int seq,
                                            float c2, int64_t b, int64_t r0, int k0, int keys,
                                            const float (&rmx)[16], const float (&rinv)[16], _Float16* ldsQ) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, l32 = lane & 31, hl = lane >> 5;
    const int np = keys / kPanelQ;
    f16x8 aq[8];                                  // A operand: row r0 + l32
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        aq[ks] = *reinterpret_cast<const f16x8*>(Q + (r0 + l32) * kD2 + ks * 16 + hl * 8);
    }
    const _Float16* kb = K + (b * seq + k0) * kD2;
    u32x4v v[8];
    loadPanelQ(kb, tid, v);
    storePanelQ(ldsQ, tid, v);
    __syncthreads();
    for (int p = 0; p < np; ++p) {
        if (p + 1 < np) loadPanelQ(kb + static_cast<int64_t>(p + 1) * kPanelQ * kD2, tid, v);
        const _Float16* pk = ldsQ + (p & 1) * kPanelHalvesQ;
        f32x16 acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f16x8 x = *reinterpret_cast<const f16x8*>(pk + (j * 32 + l32) * kRowQ + ks * 16 + hl * 8);
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aq[ks], x, acc[j], 0, 0, 0);
            }
        }
        const int kc = k0 + p * kPanelQ;
        float bj[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bj[j] = bias[kc + j * 32 + l32] * kLog2e;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float* dst = S + (r0 + 8 * (r >> 2) + 4 * hl + (r & 3)) * static_cast<int64_t>(seq) + kc + l32;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                dst[j * 32] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[j][r], c2, bj[j]) - rmx[r]) * rinv[r];
            }
        }
        if (p + 1 < np) storePanelQ(ldsQ + ((p + 1) & 1) * kPanelHalvesQ, tid, v);
        __syncthreads();
    }
}

__global__ __launch_bounds__(256, 2) void scoreStatsQ(const _Float16* __restrict__ Q,
                                                      const _Float16* __restrict__ K,
                                                      const float* __restrict__ bias,
                                                      float2* __restrict__ part, int seq, float c2) {
    extern __shared__ __align__(16) _Float16 ldsQ[];
    int64_t b;
    int rb, kh;
    blockOfQ(seq / 128, b, rb, kh);
    int64_t qrow;
    const float2 st = statsRangeQ(Q, K, bias, seq, c2, b, rb, kh * (seq / 2), seq / 2, ldsQ, qrow);
    if (((threadIdx.x & 63) >> 5) == 0) part[qrow * 2 + kh] = st;
}

__global__ __launch_bounds__(256, 2) void scoreStoreQ(const _Float16* __restrict__ Q,
                                                      const _Float16* __restrict__ K,
                                                      const float* __restrict__ bias,
                                                      const float2* __restrict__ part, float* __restrict__ S,
                                                      int seq, float c2) {
    extern __shared__ __align__(16) _Float16 ldsQ[];
    int64_t b;
    int rb, kh;
    blockOfQ(seq / 128, b, rb, kh);
    const int64_t r0 = b * seq + static_cast<int64_t>(rb) * 128 + (threadIdx.x >> 6) * 32;
    float rmx[16], rinv[16];
    mergeStatsQ<2>(part, r0, rmx, rinv);
    storeRangeQ(Q, K, bias, S, seq, c2, b, r0, kh * (seq / 2), seq / 2, rmx, rinv, ldsQ);
}

int launchQ(const mlkd_score_softmax* p, hipStream_t st) {
    const size_t ldsStats = kLdsStoreQ + static_cast<size_t>(p->seq / 2) * sizeof(float);
    static bool attrs = false;
    if (!attrs) {
        const size_t maxStats = kLdsStoreQ + static_cast<size_t>(kMaxSeqQ / 2) * sizeof(float);
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(scoreStatsQ), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(maxStats)) != hipSuccess ||
            hipFuncSetAttribute(reinterpret_cast<const void*>(scoreStoreQ), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(kLdsStoreQ)) != hipSuccess) {
            return MLKD_RT_LAUNCH;
        }
        attrs = true;
    }
    const unsigned blocks = static_cast<unsigned>(p->batch * (p->seq / 128) * 2);
    // Both passes work in base 2: v2 = acc * (log2(e) / div) + bias * log2(e),
    // exp(v - max) = exp2(v2 - max2).
    const float c2 = static_cast<float>(1.4426950408889634 / p->div);
    hipLaunchKernelGGL(scoreStatsQ, dim3(blocks), dim3(256), ldsStats, st, static_cast<const _Float16*>(p->q),
                       static_cast<const _Float16*>(p->k), static_cast<const float*>(p->bias),
                       static_cast<float2*>(p->scratch), static_cast<int>(p->seq), c2);
    hipLaunchKernelGGL(scoreStoreQ, dim3(blocks), dim3(256), kLdsStoreQ, st, static_cast<const _Float16*>(p->q),
                       static_cast<const _Float16*>(p->k), static_cast<const float*>(p->bias),
                       static_cast<const float2*>(p->scratch), static_cast<float*>(p->s), static_cast<int>(p->seq),
                       c2);
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

bool twoPassApplies(const mlkd_score_softmax* p) {
    return p->qk_dtype == MLKD_F16 && p->bias_dtype == MLKD_F32 && p->s_dtype == MLKD_F32 &&
           p->dim == kD2 && p->seq % 256 == 0 && p->seq > 0 && p->seq <= (1 << 16) &&
           (reinterpret_cast<uintptr_t>(p->q) & 15u) == 0 && (reinterpret_cast<uintptr_t>(p->k) & 15u) == 0 &&
           p->batch * (p->seq / 128) * (p->seq / 256) <= 0x7FFFFFFF;
}

/// Partials are kept per 128-key block (the smallest key block any stats
/// shape uses), so every stats shape fits the same scratch.
int64_t scratch2(const mlkd_score_softmax* p) {
    return p->batch * p->seq * (p->seq / 128) * static_cast<int64_t>(sizeof(float2));
}

template <int ROWS, int COLS, int KST>
int launchStats2(const mlkd_score_softmax* p, hipStream_t st, float rdiv) {
    using SH = Shape2<ROWS, COLS, KST>;
    static bool attr = false;
    if (!attr && SH::kLds > 65536) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(scoreStats2<ROWS, COLS, KST>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(SH::kLds)) != hipSuccess) {
            return -1;
        }
    }
    attr = true;
    const unsigned blocks = static_cast<unsigned>(p->batch * (p->seq / ROWS) * (p->seq / COLS));
    hipLaunchKernelGGL((scoreStats2<ROWS, COLS, KST>), dim3(blocks), dim3(SH::kThreads), SH::kLds, st,
                       static_cast<const _Float16*>(p->q), static_cast<const _Float16*>(p->k),
                       static_cast<const float*>(p->bias), static_cast<float2*>(p->scratch),
                       static_cast<int>(p->seq), rdiv);
    return static_cast<int>(p->seq / ROWS);
}

template <int ROWS, int COLS, int KST, bool NT>
int launchStore2(const mlkd_score_softmax* p, hipStream_t st, float rdiv, int nKB) {
    using SH = Shape2<ROWS, COLS, KST>;
    static bool attr = false;
    if (!attr && SH::kLds > 65536 - 2 * ROWS * 4) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(scoreStore2<ROWS, COLS, KST, NT>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(SH::kLds)) != hipSuccess) {
            return -1;
        }
    }
    attr = true;
    const unsigned blocks = static_cast<unsigned>(p->batch * (p->seq / ROWS) * (p->seq / COLS));
    hipLaunchKernelGGL((scoreStore2<ROWS, COLS, KST, NT>), dim3(blocks), dim3(SH::kThreads), SH::kLds, st,
                       static_cast<const _Float16*>(p->q), static_cast<const _Float16*>(p->k),
                       static_cast<const float*>(p->bias), static_cast<const float2*>(p->scratch),
                       static_cast<float*>(p->s), static_cast<int>(p->seq), nKB, rdiv);
    return 0;
}

// Two-pass forms: v8 (default) query-stationary, seq <= 8192; v3 the
// 256 x 256 block form for any seq multiple of 256.
int launchTwoPass(const mlkd_score_softmax* p, hipStream_t st, int variant) {
    if (variant != 3 && p->seq <= kMaxSeqQ) return launchQ(p, st);
    const float rdiv = static_cast<float>(1.0 / p->div);
    const int nKB = launchStats2<256, 256, 128>(p, st, rdiv);
    if (nKB < 0 || launchStore2<256, 256, 128, false>(p, st, rdiv, nKB) != 0) return MLKD_RT_LAUNCH;
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

template <typename T>
__device__ __forceinline__ double ldAny(const void* p, int dt, int64_t i) {
    if (dt == MLKD_F32) return static_cast<const float*>(p)[i];
    if (dt == MLKD_F16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
    return static_cast<const double*>(p)[i];
}

__global__ __launch_bounds__(256) void scoresGeneral(mlkd_score_softmax p) {
    const int64_t total = p.batch * p.seq * p.seq;
    for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t j = t % p.seq;
        const int64_t bi = t / p.seq;  // b*seq + i
        const int64_t b = bi / p.seq;
        double acc = 0.0;
        for (int64_t k = 0; k < p.dim; ++k) {
            acc += ldAny<double>(p.q, p.qk_dtype, bi * p.dim + k) *
                   ldAny<double>(p.k, p.qk_dtype, (b * p.seq + j) * p.dim + k);
        }
        const double v = acc / p.div + ldAny<double>(p.bias, p.bias_dtype, j);
        if (p.s_dtype == MLKD_F32) {
            static_cast<float*>(p.s)[t] = static_cast<float>(v);
        } else if (p.s_dtype == MLKD_F64) {
            static_cast<double*>(p.s)[t] = v;
        } else {
            static_cast<_Float16*>(p.s)[t] = mlk::toHalf(v);
        }
    }
}

// 0: the best form for the shape; 1: scores then softmax; 2: fused single
// pass; 3: two-pass 256 x 256 blocks; 8: two-pass query-stationary.
int gScoreVariant = 0;

}  // namespace

extern "C" void mlkd_score_set_variant(int variant) { gScoreVariant = variant; }

extern "C" int64_t mlkd_score_scratch_bytes(const mlkd_score_softmax* p) {
    return p != nullptr && twoPassApplies(p) ? scratch2(p) : 0;
}

extern "C" int mlkd_launch_score_softmax(const mlkd_score_softmax* p, void* stream) {
    if (p == nullptr || p->batch < 0 || p->seq < 0 || p->dim < 0) return MLKD_RT_LAUNCH;
    if (p->batch == 0 || p->seq == 0) return 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int variant = p->variant >= 0 ? p->variant : gScoreVariant;
    if ((variant == 0 || variant == 3 || variant == 8) && twoPassApplies(p) &&
        p->scratch != nullptr && (reinterpret_cast<uintptr_t>(p->scratch) & 7u) == 0 &&
        p->scratch_bytes >= scratch2(p)) {
        return launchTwoPass(p, st, variant);
    }
    const bool fast = p->qk_dtype == MLKD_F16 && p->bias_dtype == MLKD_F32 && p->s_dtype == MLKD_F32 &&
                      p->seq % 128 == 0 && p->dim % 16 == 0 && p->dim > 0 && p->seq < (1 << 20) &&
                      (reinterpret_cast<uintptr_t>(p->q) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(p->k) & 15u) == 0 && p->dim % 8 == 0;
    const bool fused = fast && p->seq <= 2048 && p->dim <= 256 && variant != 1;
    // Second fused form for dim 64/128 and seq a multiple of 256 (8 waves of
    // seq/256 tiles, at most 8 tiles per wave).
    if (fused && (p->dim == 128 || p->dim == 64) && p->seq % 256 == 0) {
        const int64_t blocks = p->batch * (p->seq / 32);
        if (blocks > 0x7FFFFFFF) return MLKD_RT_LAUNCH;
        const int nt = static_cast<int>(p->seq / 256);
        auto launch = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(512), 0, st,
                               static_cast<const _Float16*>(p->q), static_cast<const _Float16*>(p->k),
                               static_cast<const float*>(p->bias), static_cast<float*>(p->s),
                               static_cast<int>(p->seq), static_cast<float>(p->div));
        };
        if (p->dim == 128) {
            switch (nt) {
                case 1: launch(scoreSoftmaxFusedT<8, 1, 8>); break;
                case 2: launch(scoreSoftmaxFusedT<8, 2, 8>); break;
                case 3: launch(scoreSoftmaxFusedT<8, 3, 8>); break;
                case 4: launch(scoreSoftmaxFusedT<8, 4, 8>); break;
                case 5: launch(scoreSoftmaxFusedT<8, 5, 8>); break;
                case 6: launch(scoreSoftmaxFusedT<8, 6, 8>); break;
                case 7: launch(scoreSoftmaxFusedT<8, 7, 8>); break;
                default: launch(scoreSoftmaxFusedT<8, 8, 8>); break;
            }
        } else {
            switch (nt) {
                case 1: launch(scoreSoftmaxFusedT<8, 1, 4>); break;
                case 2: launch(scoreSoftmaxFusedT<8, 2, 4>); break;
                case 3: launch(scoreSoftmaxFusedT<8, 3, 4>); break;
                case 4: launch(scoreSoftmaxFusedT<8, 4, 4>); break;
                case 5: launch(scoreSoftmaxFusedT<8, 5, 4>); break;
                case 6: launch(scoreSoftmaxFusedT<8, 6, 4>); break;
                case 7: launch(scoreSoftmaxFusedT<8, 7, 4>); break;
                default: launch(scoreSoftmaxFusedT<8, 8, 4>); break;
            }
        }
        return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
    }
    if (fused) {
        const int64_t blocks = p->batch * (p->seq / 32);
        if (blocks > 0x7FFFFFFF) return MLKD_RT_LAUNCH;
        const int nt = static_cast<int>(p->seq / 128);
        auto launch = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                               static_cast<const _Float16*>(p->q), static_cast<const _Float16*>(p->k),
                               static_cast<const float*>(p->bias), static_cast<float*>(p->s),
                               static_cast<int>(p->seq), static_cast<int>(p->dim), static_cast<float>(p->div));
        };
        switch (nt) {
            case 1: launch(scoreSoftmaxFused<1>); break;
            case 2: launch(scoreSoftmaxFused<2>); break;
            case 3: launch(scoreSoftmaxFused<3>); break;
            case 4: launch(scoreSoftmaxFused<4>); break;
            case 5: launch(scoreSoftmaxFused<5>); break;
            case 6: launch(scoreSoftmaxFused<6>); break;
            case 7: launch(scoreSoftmaxFused<7>); break;
            case 8: launch(scoreSoftmaxFused<8>); break;
            case 9: launch(scoreSoftmaxFused<9>); break;
            case 10: launch(scoreSoftmaxFused<10>); break;
            case 11: launch(scoreSoftmaxFused<11>); break;
            case 12: launch(scoreSoftmaxFused<12>); break;
            case 13: launch(scoreSoftmaxFused<13>); break;
            case 14: launch(scoreSoftmaxFused<14>); break;
            case 15: launch(scoreSoftmaxFused<15>); break;
            default: launch(scoreSoftmaxFused<16>); break;
        }
        return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
    }
    if (fast) {
        const int64_t blocks = p->batch * (p->seq / 64) * (p->seq / 128);
        if (blocks > 0x7FFFFFFF) return MLKD_RT_LAUNCH;
        hipLaunchKernelGGL(scoresF16, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                           static_cast<const _Float16*>(p->q), static_cast<const _Float16*>(p->k),
                           static_cast<const float*>(p->bias), static_cast<float*>(p->s),
                           static_cast<int>(p->seq), static_cast<int>(p->dim), static_cast<float>(p->div));
    } else {
        hipLaunchKernelGGL(scoresGeneral, dim3(8192), dim3(256), 0, st, *p);
    }
    if (hipGetLastError() != hipSuccess) return MLKD_RT_LAUNCH;
    mlkd_softmax sm;
    sm.variant = -1;
    sm.pad = 0;
    sm.x = p->s;
    sm.y = p->s;
    sm.x_dtype = p->s_dtype;
    sm.y_dtype = p->s_dtype;
    sm.rows = p->batch * p->seq;
    sm.cols = p->seq;
    sm.x_row_stride = p->seq;
    sm.y_row_stride = p->seq;
    return mlkd_launch_softmax(&sm, stream);
}
