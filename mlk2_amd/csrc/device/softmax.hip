// Row-wise stable softmax: Call(Softmax) (runtime/src/execution/
// kernel_buffers.cpp:290-340) and the synthesized six-statement nest of
// compiler/src/passes/poly/poly.synth.cpp:363-523, which computes the same
// values through materialized temps. Per row: r = max over x (a NaN never
// replaces the running max, matching (x > r) ? x : r); y = exp(x - r);
// s = sum y; y = s != 0 ? y / s : 0. The temps are never materialized: the
// row lives in registers between its one HBM read and its one HBM write.
//
// Fast path (f32 in/out, cols % 4 == 0, cols <= 256*CH): one wave per row,
// each lane holds CH float4 of the row (16-byte coalesced loads), the max and
// the sum are wave reductions (ds_swizzle/DPP through __shfl_xor), no LDS and
// no barriers. exp runs in f32 on x - r (x - r is exact whenever x is near r,
// which is where the large outputs are); the row sum accumulates in f64, so
// the normalisation error stays ~1 f32 ULP of each output.
// General path (any dtype, any cols): one workgroup per row, three passes over
// the row with LDS reductions, f64 throughout.
#include <hip/hip_runtime.h>

#include <cstdio>

#include <math.h>
#include <stdint.h>

#include "mlk_device_math.h"
#include "runtime_abi.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float waveMax(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ double waveSum(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

/// Loads one row into the lane's CH float4 (columns past `cols` read as -inf,
/// which leaves the max unchanged and adds exp(-inf) = 0 to nothing: the sum
/// skips them). FULL: cols == 256 * CH, so every column is in range and the
/// guards compile away.
template <int CH, bool FULL>
__device__ __forceinline__ void loadRow(const float* xr, int64_t cols, int lane, f32x4 (&v)[CH]) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int64_t col = (static_cast<int64_t>(c) * 64 + lane) * 4;
        if (FULL || col < cols) {
            v[c] = *reinterpret_cast<const f32x4*>(xr + col);
        } else {
            v[c] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        }
    }
}

/// The row max, wave-reduced (every lane returns it).
template <int CH>
__device__ __forceinline__ float rowMax(const f32x4 (&v)[CH]) {
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) m = fmaxf(m, v[c][e]);
    }
    return waveMax(m);
}

/// exp(v - m), the row sum, and the stores of v / sum. FAST: exp as
/// v_exp_f32 of (x - max) * log2(e), and the row sum as f64 over f32 sums of
/// each 4-element group (the error of either stays below 1e-7 relative of the
/// result, against the class's 1e-6). NT: nontemporal stores.
template <int CH, bool FAST, bool NT, bool FULL>
__device__ __forceinline__ void normalizeRow(f32x4 (&v)[CH], float m, float* yr, int64_t cols, int lane) {
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int64_t col = (static_cast<int64_t>(c) * 64 + lane) * 4;
        if constexpr (FAST) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[c][e] = __builtin_amdgcn_exp2f((v[c][e] - m) * 1.44269504088896340736f);
            if (FULL || col < cols) s += static_cast<double>((v[c][0] + v[c][1]) + (v[c][2] + v[c][3]));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ex = expf(v[c][e] - m);
                v[c][e] = ex;
                if (FULL || col < cols) s += static_cast<double>(ex);
            }
        }
    }
    s = waveSum(s);
    // The reference's `s != 0 ? y / s : 0` never takes its zero arm here: an
    // in-range element equal to the max m contributes exp(0) = 1, and a row
    // with no such element (m = +-inf, or every element NaN) makes some term
    // NaN (inf - inf, NaN - m). So s >= 1 or s is NaN, and y * (1 / s) is
    // the reference's value without a per-element select.
    const float inv = static_cast<float>(1.0 / s);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int64_t col = (static_cast<int64_t>(c) * 64 + lane) * 4;
        if (FULL || col < cols) {
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = v[c][e] * inv;
            if constexpr (NT) {
                __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(yr + col));
            } else {
                *reinterpret_cast<f32x4*>(yr + col) = o;
            }
        }
    }
}

template <int CH, bool FAST, bool NT, bool FULL>
__device__ __forceinline__ void finishRow(f32x4 (&v)[CH], float* yr, int64_t cols, int lane) {
    normalizeRow<CH, FAST, NT, FULL>(v, rowMax<CH>(v), yr, cols, lane);
}

/// One row per wave. Always the guarded row body: the guard-free one
/// (FULL) holds 150 VGPRs here against 88, and at 3 waves per SIMD instead
/// of 5 it measured 41.3 us against 40.2 us at 8192 x 4096.
template <int CH, bool FAST = false, bool NT = true>
__global__ __launch_bounds__(256) void softmaxWaveRow(const float* x,
                                                      float* y, int64_t rows,
                                                      int64_t cols, int64_t xs, int64_t ys) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t row = wave; row < rows; row += waves) {
        f32x4 v[CH];
        loadRow<CH, false>(x + row * xs, cols, lane, v);
        finishRow<CH, FAST, NT, false>(v, y + row * ys, cols, lane);
    }
}

/// Rows the float4 loads cannot take (cols % 4 != 0, or a row start off 16
/// bytes), up to 256 * CH columns: one wave per row with the arithmetic of
/// softmaxWaveRow<CH, true, true> (f32 max, v_exp_f32, f64 sum of f32 sums
/// of 4-element groups), 4-byte loads and stores that are lane-contiguous
/// per instruction. v[c][e] holds element c * 256 + e * 64 + lane; elements
/// past the row read as -inf and add exp2(-inf) = 0 to their group.
template <int CH>
__global__ __launch_bounds__(256) void softmaxWaveRowScalar(const float* __restrict__ x, float* __restrict__ y,
                                                            int64_t rows, int64_t cols, int64_t xs, int64_t ys) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t row = wave; row < rows; row += waves) {
        const float* xr = x + row * xs;
        float* yr = y + row * ys;
        f32x4 v[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t col = static_cast<int64_t>(c) * 256 + e * 64 + lane;
                v[c][e] = col < cols ? xr[col] : -INFINITY;
            }
        }
        const float m = rowMax<CH>(v);
        double s = 0.0;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[c][e] = __builtin_amdgcn_exp2f((v[c][e] - m) * 1.44269504088896340736f);
            s += static_cast<double>((v[c][0] + v[c][1]) + (v[c][2] + v[c][3]));
        }
        s = waveSum(s);
        const float inv = static_cast<float>(1.0 / s);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t col = static_cast<int64_t>(c) * 256 + e * 64 + lane;
                if (col < cols) __builtin_nontemporal_store(v[c][e] * inv, yr + col);
            }
        }
    }
}

/// Two adjacent rows per wave: the second row's loads are issued once the
/// first row's max is known, so they land while the first row is
/// exponentiated, summed and stored. The per-row arithmetic is that of form 0
/// (rowMax, then normalizeRow<CH, true, true>), so the two forms agree bit
/// for bit.
template <int CH, bool FULL>
__global__ __launch_bounds__(256) void softmaxWaveRowPair(const float* x, float* y, int64_t rows, int64_t cols,
                                                          int64_t xs, int64_t ys) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    const int64_t pairs = (rows + 1) / 2;
    for (int64_t pr = wave; pr < pairs; pr += waves) {
        // An odd last row pairs with itself: the same wave computes it twice
        // from the same data and stores the same bits twice. A branch around
        // the second row instead makes the compiler's wait counts assume the
        // second row's loads were issued and drain them all before the first
        // row's reductions, which serialises the pair.
        const int64_t r0 = 2 * pr;
        const int64_t r1 = r0 + 1 < rows ? r0 + 1 : r0;
        f32x4 a[CH], b[CH];
        loadRow<CH, FULL>(x + r0 * xs, cols, lane, a);
        const float ma = rowMax<CH>(a);
        // The barriers fix the order (measured at 8192 x 4096: 39.3 us with
        // it, 39.7 us with both rows' loads first, 40.1 us with the rows'
        // bodies merged by the scheduler, which then waits for both rows
        // before either reduction and holds both rows' temporaries).
        __builtin_amdgcn_sched_barrier(0);
        loadRow<CH, FULL>(x + r1 * xs, cols, lane, b);
        __builtin_amdgcn_sched_barrier(0);
        normalizeRow<CH, true, true, FULL>(a, ma, y + r0 * ys, cols, lane);
        __builtin_amdgcn_sched_barrier(0);
        finishRow<CH, true, true, FULL>(b, y + r1 * ys, cols, lane);
    }
}

/// The row body of form 2 (expf, per-element f64 sums), with each wave
/// walking several rows and the next row's loads issued before the current
/// row's reductions, so HBM reads of row r+1 overlap the exp/sum/stores of
/// row r.
template <int CH>
__global__ __launch_bounds__(256) void softmaxWaveRowPipelined(const float* x, float* y, int64_t rows,
                                                               int64_t cols, int64_t xs, int64_t ys) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    f32x4 cur[CH], nxt[CH];
    if (wave < rows) loadRow<CH, false>(x + wave * xs, cols, lane, cur);
    for (int64_t row = wave; row < rows; row += waves) {
        const int64_t nrow = row + waves;
        if (nrow < rows) loadRow<CH, false>(x + nrow * xs, cols, lane, nxt);
        finishRow<CH, false, true, false>(cur, y + row * ys, cols, lane);
#pragma unroll
        for (int c = 0; c < CH; ++c) cur[c] = nxt[c];
    }
}

template <typename T>
__device__ __forceinline__ double ld(const void* p, int64_t i) {
    return static_cast<double>(static_cast<const T*>(p)[i]);
}

__device__ __forceinline__ double loadAny(const void* p, int dt, int64_t i) {
    if (dt == MLKD_F32) return ld<float>(p, i);
    if (dt == MLKD_F16) return static_cast<double>(static_cast<float>(static_cast<const _Float16*>(p)[i]));
    return ld<double>(p, i);
}

__device__ __forceinline__ void storeAny(void* p, int dt, int64_t i, double v) {
    if (dt == MLKD_F32) {
        static_cast<float*>(p)[i] = static_cast<float>(v);
    } else if (dt == MLKD_F16) {
        static_cast<_Float16*>(p)[i] = mlk::toHalf(v);
    } else {
        static_cast<double*>(p)[i] = v;
    }
}

__device__ __forceinline__ double blockReduce(double v, bool isMax, double* scratch) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const double o = __shfl_xor(v, off, 64);
        v = isMax ? ((o > v) ? o : v) : v + o;
    }
    if (lane == 0) scratch[w] = v;
    __syncthreads();
    double r = scratch[0];
    for (int i = 1; i < static_cast<int>(blockDim.x >> 6); ++i) {
        r = isMax ? ((scratch[i] > r) ? scratch[i] : r) : r + scratch[i];
    }
    __syncthreads();
    return r;
}

/// General path: any dtype, any row length. f64 arithmetic as the reference.
__global__ __launch_bounds__(256) void softmaxBlockRow(mlkd_softmax p) {
    __shared__ double scratch[4];
    for (int64_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
        const int64_t xo = row * p.x_row_stride;
        const int64_t yo = row * p.y_row_stride;
        double r = -INFINITY;
        for (int64_t c = threadIdx.x; c < p.cols; c += blockDim.x) {
            const double v = loadAny(p.x, p.x_dtype, xo + c);
            r = (v > r) ? v : r;
        }
        r = blockReduce(r, true, scratch);
        double s = 0.0;
        for (int64_t c = threadIdx.x; c < p.cols; c += blockDim.x) {
            s += exp(loadAny(p.x, p.x_dtype, xo + c) - r);
        }
        s = blockReduce(s, false, scratch);
        for (int64_t c = threadIdx.x; c < p.cols; c += blockDim.x) {
            const double e = exp(loadAny(p.x, p.x_dtype, xo + c) - r);
            storeAny(p.y, p.y_dtype, yo + c, s != 0.0 ? e / s : 0.0);
        }
    }
}

// Launch variant of the wave-per-row path. 0: one row per wave, v_exp_f32 and
// grouped sums, nontemporal stores; 1: rows pipelined over a grid of
// `gSoftmaxWaves` waves; 2: as 0 with the accurate expf and per-element f64
// sums; 3: as 0 with plain stores; 4: as 2 with plain stores; 5: as 0 with two
// adjacent rows per wave (the default: on gfx950 at 8192 x 4096, 38.9 us
// against 39.8 us for form 0 and 37.4 us for a copy of the same bytes). Set
// by the variant search (mlkd_softmax_set_variant).
int gSoftmaxVariant = 5;
int64_t gSoftmaxWaves = 0;

template <int CH>
int launchWave(const mlkd_softmax& p, hipStream_t st) {
    const int variant = p.variant >= 0 ? p.variant : gSoftmaxVariant;
    if (variant == 1) {
        int64_t waves = gSoftmaxWaves > 0 ? gSoftmaxWaves : 2048;
        if (waves > p.rows) waves = p.rows;
        const int64_t blocks = (waves + 3) / 4;
        hipLaunchKernelGGL(softmaxWaveRowPipelined<CH>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                           static_cast<const float*>(p.x), static_cast<float*>(p.y), p.rows, p.cols,
                           p.x_row_stride, p.y_row_stride);
        return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
    }
    const bool full = p.cols == 256 * CH;
    if (variant == 5) {
        int64_t blocks = ((p.rows + 1) / 2 + 3) / 4;
        if (blocks > 8192) blocks = 8192;
        auto pair = full ? softmaxWaveRowPair<CH, true> : softmaxWaveRowPair<CH, false>;
        hipLaunchKernelGGL(pair, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                           static_cast<const float*>(p.x), static_cast<float*>(p.y), p.rows, p.cols,
                           p.x_row_stride, p.y_row_stride);
        return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
    }
    int64_t blocks = (p.rows + 3) / 4;
    if (gSoftmaxWaves > 0 && blocks > (gSoftmaxWaves + 3) / 4) blocks = (gSoftmaxWaves + 3) / 4;
    if (blocks > 8192) blocks = 8192;
    auto kern = softmaxWaveRow<CH, true, true>;
    if (variant == 2) kern = softmaxWaveRow<CH, false, true>;
    if (variant == 3) kern = softmaxWaveRow<CH, true, false>;
    if (variant == 4) kern = softmaxWaveRow<CH, false, false>;
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, static_cast<const float*>(p.x),
                       static_cast<float*>(p.y), p.rows, p.cols, p.x_row_stride, p.y_row_stride);
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

template <int CH>
int launchScalar(const mlkd_softmax& p, hipStream_t st) {
    int64_t blocks = (p.rows + 3) / 4;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(softmaxWaveRowScalar<CH>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       static_cast<const float*>(p.x), static_cast<float*>(p.y), p.rows, p.cols, p.x_row_stride,
                       p.y_row_stride);
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

/// f32 rows up to 8192 columns that the float4 path does not take.
bool scalarApplies(const mlkd_softmax* p) {
    return p->x_dtype == MLKD_F32 && p->y_dtype == MLKD_F32 && p->cols <= 8192 &&
           (reinterpret_cast<uintptr_t>(p->x) & 3u) == 0 && (reinterpret_cast<uintptr_t>(p->y) & 3u) == 0;
}

}  // namespace

extern "C" void mlkd_softmax_set_variant(int variant, int64_t waves) {
    gSoftmaxVariant = variant;
    gSoftmaxWaves = waves;
}

extern "C" const char* mlkd_softmax_kernel_name(const mlkd_softmax* p) {
    static thread_local char name[96];
    const bool aligned = (reinterpret_cast<uintptr_t>(p->x) & 15u) == 0 &&
                         (reinterpret_cast<uintptr_t>(p->y) & 15u) == 0 &&
                         (p->x_row_stride & 3) == 0 && (p->y_row_stride & 3) == 0;
    int ch = 1;
    while (256 * ch < p->cols) ch *= 2;
    if (!(p->x_dtype == MLKD_F32 && p->y_dtype == MLKD_F32 && (p->cols & 3) == 0 && aligned && p->cols <= 8192)) {
        if (!scalarApplies(p)) return "softmaxBlockRow";
        std::snprintf(name, sizeof(name), "softmaxWaveRowScalar<%d>", ch);
        return name;
    }
    const int variant = p->variant >= 0 ? p->variant : gSoftmaxVariant;
    if (variant == 1) {
        std::snprintf(name, sizeof(name), "softmaxWaveRowPipelined<%d>", ch);
    } else if (variant == 5) {
        std::snprintf(name, sizeof(name), "softmaxWaveRowPair<%d, %s>", ch, p->cols == 256 * ch ? "true" : "false");
    } else {
        const bool fastExp = variant != 2 && variant != 4, nt = variant != 3 && variant != 4;
        std::snprintf(name, sizeof(name), "softmaxWaveRow<%d, %s, %s>", ch, fastExp ? "true" : "false",
                      nt ? "true" : "false");
    }
    return name;
}

extern "C" int mlkd_launch_softmax(const mlkd_softmax* p, void* stream) {
    if (p == nullptr || p->rows < 0 || p->cols < 0) return MLKD_RT_LAUNCH;
    if (p->rows == 0 || p->cols == 0) return 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool aligned = (reinterpret_cast<uintptr_t>(p->x) & 15u) == 0 &&
                         (reinterpret_cast<uintptr_t>(p->y) & 15u) == 0 &&
                         (p->x_row_stride & 3) == 0 && (p->y_row_stride & 3) == 0;
    if (p->x_dtype == MLKD_F32 && p->y_dtype == MLKD_F32 && (p->cols & 3) == 0 && aligned) {
        if (p->cols <= 256) return launchWave<1>(*p, st);
        if (p->cols <= 512) return launchWave<2>(*p, st);
        if (p->cols <= 1024) return launchWave<4>(*p, st);
        if (p->cols <= 2048) return launchWave<8>(*p, st);
        if (p->cols <= 4096) return launchWave<16>(*p, st);
        if (p->cols <= 8192) return launchWave<32>(*p, st);
    }
    if (scalarApplies(p)) {
        if (p->cols <= 256) return launchScalar<1>(*p, st);
        if (p->cols <= 512) return launchScalar<2>(*p, st);
        if (p->cols <= 1024) return launchScalar<4>(*p, st);
        if (p->cols <= 2048) return launchScalar<8>(*p, st);
        if (p->cols <= 4096) return launchScalar<16>(*p, st);
        return launchScalar<32>(*p, st);
    }
    int64_t blocks = p->rows < 65536 ? p->rows : 65536;
    hipLaunchKernelGGL(softmaxBlockRow, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, *p);
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

namespace {

/// Row sum (Call(ReduceSum), kernel_buffers.cpp:237-277, and the poly.synth
/// ReduceSum nest): one wave per row, f64 accumulation (strided per lane,
/// then a wave reduction).
__global__ __launch_bounds__(256) void rowSumWave(mlkd_softmax p) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t row = wave; row < p.rows; row += waves) {
        double s = 0.0;
        for (int64_t c = lane; c < p.cols; c += 64) s += loadAny(p.x, p.x_dtype, row * p.x_row_stride + c);
        s = waveSum(s);
        if (lane == 0) storeAny(p.y, p.y_dtype, row * p.y_row_stride, s);
    }
}

}  // namespace

extern "C" int mlkd_launch_rowsum(const mlkd_softmax* p, void* stream) {
    if (p == nullptr || p->rows < 0 || p->cols < 0) return MLKD_RT_LAUNCH;
    if (p->rows == 0) return 0;
    int64_t blocks = (p->rows + 3) / 4;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(rowSumWave, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), *p);
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}
