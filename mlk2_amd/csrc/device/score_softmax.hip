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
//   * scores, then the softmax kernel in place over S (any shape, f16);
//   * a scalar f64 path for other dtypes.
#include <hip/hip_runtime.h>

#include <cstdio>

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

// ------------------------------------------------------------ two pass ----
constexpr int kD2 = 128;                 // head dim
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

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
//   exp2(v - (max + log2 sum)) for the panel at once: each 32-lane half-wave
//   stores one 128-byte line, while the other workgroup on the CU computes.
// Both passes work in base 2 with log2(e) folded into 1/div and the bias, so
// a score costs one fused multiply-add and one v_exp_f32. Pass 2 is bound by
// its stores (256 MiB in the MFMA output layout); pass 1 by its MFMAs and
// the VALU work per score together.
constexpr int kPanelQ = 128;                   // keys per streamed panel
constexpr float kLog2e = 1.44269504088896340736f;
constexpr int kRowQ = kD2 + 8;                 // halves per LDS panel row
constexpr int kPanelHalvesQ = kPanelQ * kRowQ;
constexpr size_t kLdsStoreQ = 2 * kPanelHalvesQ * sizeof(_Float16);  // pass 1 adds seq/2 floats of bias
constexpr int64_t kMaxSeqQ = 8192;             // pass 1's LDS stays <= 86 KiB

/// The max to subtract before exp2: a max of -inf (every score so far -inf)
/// is replaced by 0, so those scores contribute exp2(-inf) = 0 rather than
/// exp2(-inf - -inf) = NaN; the stored max stays -inf.
__device__ __forceinline__ float finiteOr0(float m) { return m == -INFINITY ? 0.0f : m; }

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
        // A panel whose scores are all -inf adds nothing: its exponentials
        // are taken against a finite stand-in for the -inf max.
        const float mn = fmaxf(m, mb);
        const float ms = finiteOr0(mn);
        float sb = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sb += __builtin_amdgcn_exp2f(acc[i][r] - ms);
        }
        l = l * __builtin_amdgcn_exp2f(m - ms) + sb;
        m = mn;
        if (p + 1 < np) storePanelQ(ldsQ + ((p + 1) & 1) * kPanelHalvesQ, tid, v);
        __syncthreads();
    }
    const float mo = __shfl_xor(m, 32, 64);
    const float lo = __shfl_xor(l, 32, 64);
    const float mx = fmaxf(m, mo);
    const float ms = finiteOr0(mx);
    const float lt = l * __builtin_amdgcn_exp2f(m - ms) + lo * __builtin_amdgcn_exp2f(mo - ms);
    return make_float2(mx, lt);
}

/// Row statistics of the 16 rows this lane's pass-2 accumulators hold,
/// merged from NP key-range partials part[row * NP + i] (base 2), as one
/// log-normalizer per row: rlm = max + log2(sum(exp2(v - max))), so pass 2
/// writes exp2(v - rlm) = exp2(v - max) / sum with no multiply. A row whose
/// scores are all -inf gets rlm = -inf (max -inf, sum 0): exp2(-inf - -inf)
/// writes NaN, as the reference does.
template <int NP>
__device__ __forceinline__ void mergeStatsQ(const float2* __restrict__ part, int64_t r0, float (&rlm)[16]) {
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
        const float ms = finiteOr0(mx);
        float lt = 0.0f;
#pragma unroll
        for (int i = 0; i < NP; ++i) lt += pp[i].y * __builtin_amdgcn_exp2f(pp[i].x - ms);
        rlm[r] = mx + __builtin_amdgcn_logf(lt);   // v_log_f32: log2
    }
}

/// Pass 2 over keys [k0, k0 + keys) of this wave's 32 rows r0..r0+31 of
/// batch b: D = Q K^T per panel, written as exp2(v - max) / sum at once;
/// each 32-lane half-wave stores one 128-byte line. RAGGED: Q, K and the
/// bias are zero-padded copies of length seq of a sequence of length sseq;
/// S is [batch][sseq][sseq] and only rows and keys below sseq are stored.
template <bool RAGGED>
__device__ __forceinline__ void storeRangeQ(const _Float16* __restrict__ Q, const _Float16* __restrict__ K,
                                            const float* __restrict__ bias, float* __restrict__ S, int seq,
                                            int sseq, float c2, int64_t b, int64_t r0, int k0, int keys,
                                            const float (&rlm)[16], _Float16* ldsQ) {
    const int ld = RAGGED ? sseq : seq;           // S row length
    const int i0 = static_cast<int>(r0 - b * seq);   // first row within the batch
    const int tid = threadIdx.x;
    const int lane = tid & 63, l32 = lane & 31, hl = lane >> 5;
    const int np = keys / kPanelQ;
    f16x8 aq[8];                                  // A operand: row r0 + l32
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        aq[ks] = *reinterpret_cast<const f16x8*>(Q + (r0 + l32) * kD2 + ks * 16 + hl * 8);
    }
    const _Float16* kb = K + (b * seq + k0) * kD2;
    // Stores: a scalar base per panel (row r0, key kc) plus a fixed lane
    // offset per accumulator register r, the key sub-block j as an immediate.
    uint32_t soff[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        soff[r] = static_cast<uint32_t>(((8 * (r >> 2) + 4 * hl + (r & 3)) * ld + l32) * sizeof(float));
    }
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
        char* sb = reinterpret_cast<char*>(S + (b * ld + i0) * static_cast<int64_t>(ld) + kc);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (RAGGED && (i0 + 8 * (r >> 2) + 4 * hl + (r & 3) >= sseq || kc + j * 32 + l32 >= sseq)) continue;
                *reinterpret_cast<float*>(sb + soff[r] + j * 32 * sizeof(float)) =
                    __builtin_amdgcn_exp2f(__builtin_fmaf(acc[j][r], c2, bj[j]) - rlm[r]);
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

template <bool RAGGED>
__global__ __launch_bounds__(256, 2) void scoreStoreQ(const _Float16* __restrict__ Q,
                                                      const _Float16* __restrict__ K,
                                                      const float* __restrict__ bias,
                                                      const float2* __restrict__ part, float* __restrict__ S,
                                                      int seq, int sseq, float c2) {
    extern __shared__ __align__(16) _Float16 ldsQ[];
    int64_t b;
    int rb, kh;
    blockOfQ(seq / 128, b, rb, kh);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int64_t r0 = b * seq + static_cast<int64_t>(rb) * 128 + wave * 32;   // wave-uniform
    float rlm[16];
    mergeStatsQ<2>(part, r0, rlm);
    storeRangeQ<RAGGED>(Q, K, bias, S, seq, sseq, c2, b, r0, kh * (seq / 2), seq / 2, rlm, ldsQ);
}

/// Both passes over p's (padded) Q, K and bias; `ragged` > 0 stores only
/// rows and keys below it into p->s laid out [batch][ragged][ragged].
int launchQ(const mlkd_score_softmax* p, hipStream_t st, int64_t ragged = 0) {
    const size_t ldsStats = kLdsStoreQ + static_cast<size_t>(p->seq / 2) * sizeof(float);
    // Once per process; a function-local static initializes thread-safely.
    static const bool attrs = [] {
        const size_t maxStats = kLdsStoreQ + static_cast<size_t>(kMaxSeqQ / 2) * sizeof(float);
        return hipFuncSetAttribute(reinterpret_cast<const void*>(scoreStatsQ), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   static_cast<int>(maxStats)) == hipSuccess &&
               hipFuncSetAttribute(reinterpret_cast<const void*>(scoreStoreQ<false>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsStoreQ)) == hipSuccess &&
               hipFuncSetAttribute(reinterpret_cast<const void*>(scoreStoreQ<true>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsStoreQ)) == hipSuccess;
    }();
    if (!attrs) return MLKD_RT_LAUNCH;
    const unsigned blocks = static_cast<unsigned>(p->batch * (p->seq / 128) * 2);
    // Both passes work in base 2: v2 = acc * (log2(e) / div) + bias * log2(e),
    // exp(v - max) = exp2(v2 - max2).
    const float c2 = static_cast<float>(1.4426950408889634 / p->div);
    hipLaunchKernelGGL(scoreStatsQ, dim3(blocks), dim3(256), ldsStats, st, static_cast<const _Float16*>(p->q),
                       static_cast<const _Float16*>(p->k), static_cast<const float*>(p->bias),
                       static_cast<float2*>(p->scratch), static_cast<int>(p->seq), c2);
    hipLaunchKernelGGL(ragged > 0 ? scoreStoreQ<true> : scoreStoreQ<false>, dim3(blocks), dim3(256), kLdsStoreQ, st,
                       static_cast<const _Float16*>(p->q), static_cast<const _Float16*>(p->k),
                       static_cast<const float*>(p->bias), static_cast<const float2*>(p->scratch),
                       static_cast<float*>(p->s), static_cast<int>(p->seq),
                       static_cast<int>(ragged > 0 ? ragged : p->seq), c2);
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

bool twoPassApplies(const mlkd_score_softmax* p) {
    return p->qk_dtype == MLKD_F16 && p->bias_dtype == MLKD_F32 && p->s_dtype == MLKD_F32 &&
           p->dim == kD2 && p->seq % 256 == 0 && p->seq > 0 && p->seq <= kMaxSeqQ &&
           (reinterpret_cast<uintptr_t>(p->q) & 15u) == 0 && (reinterpret_cast<uintptr_t>(p->k) & 15u) == 0 &&
           p->batch * (p->seq / 128) * 2 <= 0x7FFFFFFF;
}

/// Row statistics partials: one (max, sum) pair per row and key half.
int64_t scratch2(const mlkd_score_softmax* p) {
    return p->batch * p->seq * 2 * static_cast<int64_t>(sizeof(float2));
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

/// [batch][rows][128] f16 -> [batch][drows][128], zero rows past `rows`, in
/// 16-byte pieces (16 per row).
__global__ __launch_bounds__(256) void padQK(const u32x4v* __restrict__ src, int64_t batch, int64_t rows,
                                             u32x4v* __restrict__ dst, int64_t drows) {
    const int64_t total = batch * drows * 16;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t piece = t & 15, r = t >> 4;
        const int64_t b = r / drows, i = r % drows;
        dst[t] = i < rows ? src[(b * rows + i) * 16 + piece] : u32x4v{0u, 0u, 0u, 0u};
    }
}

/// bias' = bias on [0, seq), -inf on [seq, dseq): padded keys take no share.
__global__ __launch_bounds__(256) void padBias(const float* __restrict__ src, int64_t seq, float* __restrict__ dst,
                                               int64_t dseq) {
    for (int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; j < dseq;
         j += static_cast<int64_t>(gridDim.x) * 256) {
        dst[j] = j < seq ? src[j] : -INFINITY;
    }
}

/// The padded two-pass launch: sequence length rounded up to 256 (at most
/// kMaxSeqQ), for shapes the two passes would take but for the length.
/// Q, K and the bias are copied into the workspace (q.s stays the caller's
/// S: pass 2 stores only its rows and keys). It is faster than the general
/// kernels at every size measured, down to 1x100x128 (general: 41 us).
bool padScore(const mlkd_score_softmax* p, mlkd_score_softmax& q) {
    if (p->work == nullptr || p->seq % 256 == 0) return false;
    q = *p;
    q.seq = (p->seq + 255) / 256 * 256;
    if (q.seq > kMaxSeqQ) return false;
    unsigned char* w = static_cast<unsigned char*>(p->work);
    const size_t qk = static_cast<size_t>(p->batch * q.seq * kD2) * sizeof(_Float16);
    q.q = w;
    q.k = w + qk;
    q.bias = w + 2 * qk;
    q.scratch = w + 2 * qk + static_cast<size_t>(q.seq) * sizeof(float);
    q.scratch_bytes = scratch2(&q);
    q.work = nullptr;
    q.work_bytes = 0;
    const int64_t need = static_cast<int64_t>(2 * qk + static_cast<size_t>(q.seq) * sizeof(float)) + q.scratch_bytes;
    return twoPassApplies(&q) && p->work_bytes >= need && (reinterpret_cast<uintptr_t>(p->q) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(p->k) & 15u) == 0;
}

int launchPaddedQ(const mlkd_score_softmax* p, const mlkd_score_softmax& q, hipStream_t st) {
    const int64_t pieces = p->batch * q.seq * 16;
    const unsigned g = static_cast<unsigned>(std::min<int64_t>((pieces + 255) / 256, 16384));
    hipLaunchKernelGGL(padQK, dim3(g), dim3(256), 0, st, static_cast<const u32x4v*>(p->q), p->batch, p->seq,
                       static_cast<u32x4v*>(const_cast<void*>(q.q)), q.seq);
    hipLaunchKernelGGL(padQK, dim3(g), dim3(256), 0, st, static_cast<const u32x4v*>(p->k), p->batch, p->seq,
                       static_cast<u32x4v*>(const_cast<void*>(q.k)), q.seq);
    hipLaunchKernelGGL(padBias, dim3(static_cast<unsigned>((q.seq + 255) / 256)), dim3(256), 0, st,
                       static_cast<const float*>(p->bias), p->seq, static_cast<float*>(const_cast<void*>(q.bias)),
                       q.seq);
    if (hipGetLastError() != hipSuccess) return MLKD_RT_LAUNCH;
    return launchQ(&q, st, p->seq);
}

// 0: the best form for the shape (the two-pass query-stationary form where
// it applies); 1: scores, then the softmax kernel in place over S.
int gScoreVariant = 0;

}  // namespace

extern "C" void mlkd_score_set_variant(int variant) { gScoreVariant = variant; }

extern "C" int64_t mlkd_score_scratch_bytes(const mlkd_score_softmax* p) {
    return p != nullptr && twoPassApplies(p) ? scratch2(p) : 0;
}

extern "C" int64_t mlkd_score_pad_bytes(const mlkd_score_softmax* p) {
    if (p == nullptr) return 0;
    mlkd_score_softmax probe = *p;
    probe.work = reinterpret_cast<void*>(uintptr_t{1} << 12);
    probe.work_bytes = INT64_MAX;
    mlkd_score_softmax q;
    if (!padScore(&probe, q)) return 0;
    const int64_t qk = p->batch * q.seq * kD2 * static_cast<int64_t>(sizeof(_Float16));
    return 2 * qk + q.seq * static_cast<int64_t>(sizeof(float)) + scratch2(&q);
}

extern "C" const char* mlkd_score_kernel_names(const mlkd_score_softmax* p) {
    static thread_local char name[160];
    const int variant = p->variant >= 0 ? p->variant : gScoreVariant;
    if (mlkd_score_softmax q; variant != 1 && padScore(p, q)) return "scoreStatsQ+scoreStoreQ";
    if (variant != 1 && twoPassApplies(p) && p->scratch != nullptr &&
        (reinterpret_cast<uintptr_t>(p->scratch) & 7u) == 0 && p->scratch_bytes >= scratch2(p)) {
        return "scoreStatsQ+scoreStoreQ";
    }
    const bool fast = p->qk_dtype == MLKD_F16 && p->bias_dtype == MLKD_F32 && p->s_dtype == MLKD_F32 &&
                      p->seq % 128 == 0 && p->dim % 16 == 0 && p->dim > 0 && p->seq < (1 << 20) &&
                      (reinterpret_cast<uintptr_t>(p->q) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(p->k) & 15u) == 0 && p->dim % 8 == 0;
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
    std::snprintf(name, sizeof(name), "%s+%s", fast ? "scoresF16" : "scoresGeneral", mlkd_softmax_kernel_name(&sm));
    return name;
}

extern "C" int mlkd_launch_score_softmax(const mlkd_score_softmax* p, void* stream) {
    if (p == nullptr || p->batch < 0 || p->seq < 0 || p->dim < 0) return MLKD_RT_LAUNCH;
    if (p->batch == 0 || p->seq == 0) return 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int variant = p->variant >= 0 ? p->variant : gScoreVariant;
    if (variant != 1 && twoPassApplies(p) && p->scratch != nullptr &&
        (reinterpret_cast<uintptr_t>(p->scratch) & 7u) == 0 && p->scratch_bytes >= scratch2(p)) {
        return launchQ(p, st);
    }
    if (mlkd_score_softmax q; variant != 1 && padScore(p, q)) return launchPaddedQ(p, q, st);
    const bool fast = p->qk_dtype == MLKD_F16 && p->bias_dtype == MLKD_F32 && p->s_dtype == MLKD_F32 &&
                      p->seq % 128 == 0 && p->dim % 16 == 0 && p->dim > 0 && p->seq < (1 << 20) &&
                      (reinterpret_cast<uintptr_t>(p->q) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(p->k) & 15u) == 0 && p->dim % 8 == 0;
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
