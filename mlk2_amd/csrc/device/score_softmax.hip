// Config-5 class: S[b*seq + i, :] = softmax((Q[b,i,:] . K[b,:,:]^T) / div +
// bias), the composition of Call(MatMul) (kernel_buffers.cpp:406-432), the
// broadcast elementwise chain Add(Div(S, c), bias[j]) (poly.synth.cpp:
// 231-353) and the stable softmax (kernel_buffers.cpp:290-340).
//
// Scores: v_mfma_f32_32x32x16_f16. Both MFMA operands come straight from HBM
// with 16-byte loads: Q rows are k-contiguous, and K rows are exactly the
// columns of K^T, also k-contiguous, so no transpose is needed. A workgroup
// of 4 waves computes a 64 (i) x 128 (j) block, each wave 32 x 64; the
// epilogue divides by `div`, adds bias[j] and writes f32 scores into S. The
// softmax then runs in place over the rows of S with the wave-per-row kernel.
// Other shapes or dtypes run a scalar f64 path with the same two stages.
#include <hip/hip_runtime.h>

#include <stdint.h>

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
            static_cast<_Float16*>(p.s)[t] = static_cast<_Float16>(static_cast<float>(v));
        }
    }
}

// 0: fused single pass where the shape allows it; 1: scores then softmax.
int gScoreVariant = 0;

}  // namespace

extern "C" void mlkd_score_set_variant(int variant) { gScoreVariant = variant; }

extern "C" int mlkd_launch_score_softmax(const mlkd_score_softmax* p, void* stream) {
    if (p == nullptr || p->batch < 0 || p->seq < 0 || p->dim < 0) return MLKD_RT_LAUNCH;
    if (p->batch == 0 || p->seq == 0) return 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool fast = p->qk_dtype == MLKD_F16 && p->bias_dtype == MLKD_F32 && p->s_dtype == MLKD_F32 &&
                      p->seq % 128 == 0 && p->dim % 16 == 0 && p->dim > 0 && p->seq < (1 << 20) &&
                      (reinterpret_cast<uintptr_t>(p->q) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(p->k) & 15u) == 0 && p->dim % 8 == 0;
    const bool fused = fast && p->seq <= 2048 && p->dim <= 256 && gScoreVariant == 0;
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
