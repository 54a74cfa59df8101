// Dense C[M,N] (+)= A[M,K] * B[K,N], row-major: Call(MatMul)
// (runtime/src/execution/kernel_buffers.cpp:406-432, C accumulated in place)
// and the poly.synth init+accumulate nest (compiler/src/passes/poly/
// poly.synth.cpp:58-147, C = 0 then +=).
//
// f16 x f16 -> f32 (tensor_f16_gpu), 256x256 workgroup tiles, launch forms 0-8.
// The default, form 8 (gemmF16Dma8s, or gemmF16Dma8 when a lane offset
// needs more than 32 bits), moves both operands global -> LDS by
// the direct path into a 4-deep ring of K steps and runs 8 waves of
// v_mfma_f32_16x16x32_f16 tiles; form 7 (gemmF16Dma) is the same data path
// with 4 waves of 32x32x16 tiles. Form 0, the first: v_mfma_f32_32x32x16_f16,
// K step 64, 512 threads = 8 waves as 2 (M) x 4 (N); each wave owns
// 128x64 = 4x2 MFMA tiles (128 accumulator VGPRs). A and B tiles are double
// buffered in LDS (2 x 72 KiB): the next K step's global loads are issued
// before the current step's MFMAs and written to the other buffer after
// them, one barrier per step. A is stored as loaded ([m][k], k contiguous);
// B is transposed in registers on its way to LDS ([n][k]) so that both MFMA
// operands are single 16-byte LDS reads (8 consecutive k per lane). Rows of
// both LDS tiles are padded by 16 bytes. Workgroups are mapped XCD-aware:
// consecutive workgroup ids go to different XCDs, so the 32 tiles one XCD
// runs form a 4x8 block that shares A and B panels in that XCD's L2.
//
// f32 x f32 -> f32: v_mfma_f32_32x32x2_f32, 64x64 tiles (256 tiles at 1024^2
// fill the 256 CUs). Form 0 (K a multiple of 64, the default) moves both
// tiles by the direct path into a 4-deep LDS ring; form 1 (K a multiple of
// 32) stages them through registers, A transposed into LDS ([k][m]) and B
// stored as loaded ([k][n]) so each MFMA operand is one conflict-free 4-byte
// read.
//
// Any other shape or dtype mix runs the general tiled kernel (f32 or f64
// accumulation, bounds-checked).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>

#include "mlk_device_math.h"
#include "runtime_abi.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- f16 ----
constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kPadK = kBK + 8;           // halves per LDS row (16-byte pad)
constexpr int kTileHalves = 256 * kPadK;  // one LDS tile (A or B)

/// Skip-zero-A Call form (kernel_buffers.cpp:406-432 skips A[i,p] == 0):
/// the skip changes a result beyond the sign of a zero sum only where B
/// holds an infinity or a NaN, since 0 * inf and 0 * NaN are NaN, and then
/// every accumulator of that column is non-finite (inf * a or 0 * inf; finite
/// f16 products cannot overflow f32). So after the MFMA loop a wave checks
/// its own accumulators for an infinity or a NaN. A wave that finds one
/// recomputes its block exactly (exactWaveBlock); the
/// others store the MFMA result. f32 operands can also overflow to inf from
/// finite values; those blocks take the exact path too, which computes the
/// same overflow.
template <typename V, int I, int J>
__device__ __forceinline__ bool waveNonFinite(const V (&acc)[I][J]) {
    constexpr int E = sizeof(V) / sizeof(float);
    // A class test per value into a lane mask: no vector registers beyond
    // the accumulators, which the 4-wave forms hold in all 512.
    bool bad = false;
#pragma unroll
    for (int i = 0; i < I; ++i) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
#pragma unroll
            for (int e = 0; e < E; ++e) bad |= !__builtin_isfinite(acc[i][j][e]);
        }
    }
    return __builtin_amdgcn_ballot_w64(bad) != 0;
}

template <typename V>
__device__ __forceinline__ bool waveNonFinite(const V& acc) {
    const V one[1][1] = {{acc}};
    return waveNonFinite(one);
}

/// The exact Call(MatMul) form over one wave's rows x cols block: C_in (when
/// accumulating) plus A[i,p] * B[p,j] over p ascending, skipping A[i,p] ==
/// 0, in f32 with separate multiply and add, as the general kernel computes
/// it. Lane l takes column c0 + cb + l; rows go 4 at a time. Only a block
/// whose MFMA accumulators met a non-finite value runs it.
template <typename TA, typename TB>
__device__ __forceinline__ void exactWaveBlock(const TA* __restrict__ A, const TB* __restrict__ B,
                                               float* __restrict__ C, int64_t lda, int64_t ldb, int64_t ldc,
                                               int K, int64_t r0, int64_t c0, int rows, int cols, bool acc) {
    const int lane = threadIdx.x & 63;
    for (int cb = 0; cb < cols; cb += 64) {
        const bool on = cb + lane < cols;
        const int64_t c = c0 + cb + lane;
        for (int rb = 0; rb < rows; rb += 4) {
            float s[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = (acc && on) ? C[(r0 + rb + r) * ldc + c] : 0.0f;
            for (int k = 0; k < K; ++k) {
                const float b = on ? static_cast<float>(B[k * ldb + c]) : 0.0f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a = static_cast<float>(A[(r0 + rb + r) * lda + k]);
                    if (a != 0.0f) s[r] = s[r] + a * b;
                }
            }
            if (on) {
#pragma unroll
                for (int r = 0; r < 4; ++r) C[(r0 + rb + r) * ldc + c] = s[r];
            }
        }
    }
}

__device__ __forceinline__ void xcdTile(int tilesM, int tilesN, int& tm, int& tn) {
    const int id = blockIdx.x;
    const int total = tilesM * tilesN;
    // Group tiles 4 (M) x 8 (N) per XCD when the grid is a multiple of that.
    if (tilesM % 4 == 0 && tilesN % 8 == 0 && total % 256 == 0) {
        const int xcd = id % 8;
        const int local = id / 8;            // 0 .. total/8-1
        const int groupsN = tilesN / 8;
        const int roundTiles = 256;          // 8 XCDs x 32 tiles per round
        const int round = (id / roundTiles);
        const int localInRound = local % 32;
        const int groupId = round * 8 + xcd;
        const int gm = groupId / groupsN;
        const int gn = groupId % groupsN;
        tm = gm * 4 + localInRound / 8;
        tn = gn * 8 + localInRound % 8;
        return;
    }
    tm = id / tilesN;
    tn = id % tilesN;
}

template <bool ACC>
__global__ __launch_bounds__(512) void gemmF16Mfma(const _Float16* __restrict__ A,
                                                   const _Float16* __restrict__ B,
                                                   float* __restrict__ C, int M, int N, int K,
                                                   int64_t lda, int64_t ldb, int64_t ldc,
                                                   int /*accumulate: template ACC*/, int skipZeroA) {
    extern __shared__ __align__(16) _Float16 lds[];
    _Float16* As = lds;                      // [2][256][kPadK]
    _Float16* Bs = lds + 2 * kTileHalves;    // [2][256][kPadK]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 2;   // 0..1
    const int wn = wave & 3;    // 0..3
    int tm, tn;
    xcdTile(M / kBM, N / kBN, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kBM;
    const int64_t col0 = static_cast<int64_t>(tn) * kBN;

    // Loader roles: threads 0..255 load A (8 x 16 B each), 256..511 load a
    // 8 (k) x 8 (n) block of B each.
    const bool loadsA = tid < 256;
    const int t = tid & 255;
    // k-block fastest across lanes: the 8 lanes that share an n-block
    // write one LDS row's 8 chunks, so transposed writes are conflict-free.
    const int bk = t & 7;      // B block: k rows bk*8 .. +7
    const int bn = t >> 3;     // B block: n cols bn*8 .. +7
    u32x4 reg[8];

    auto globalLoad = [&](int k0) {
        if (loadsA) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = j * 256 + t;      // 16-byte chunk of the 256x64 tile
                const int r = c >> 3;
                const int ch = c & 7;
                reg[j] = *reinterpret_cast<const u32x4*>(A + (row0 + r) * lda + k0 + ch * 8);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                reg[r] = *reinterpret_cast<const u32x4*>(B + static_cast<int64_t>(k0 + bk * 8 + r) * ldb +
                                                        col0 + bn * 8);
            }
        }
    };
    auto ldsStore = [&](int buf) {
        if (loadsA) {
            _Float16* dst = As + buf * kTileHalves;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = j * 256 + t;
                const int r = c >> 3;
                const int ch = c & 7;
                *reinterpret_cast<u32x4*>(dst + r * kPadK + ch * 8) = reg[j];
            }
        } else {
            _Float16* dst = Bs + buf * kTileHalves;
            // 8x8 transpose of 16-bit values: column n of the block becomes
            // 8 consecutive k values.
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const int p = n >> 1;
                const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
                u32x4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    o[j] = __builtin_amdgcn_perm(reg[2 * j + 1][p], reg[2 * j][p], sel);
                }
                *reinterpret_cast<u32x4*>(dst + (bn * 8 + n) * kPadK + bk * 8) = o;
            }
        }
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
    }

    const int steps = K / kBK;
    globalLoad(0);
    ldsStore(0);
    __syncthreads();
    const int lrow = lane & 31;
    const int lk = (lane >> 5) * 8;
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        if (s + 1 < steps) globalLoad((s + 1) * kBK);
        const _Float16* as = As + buf * kTileHalves + (wm * 128 + lrow) * kPadK + lk;
        const _Float16* bs = Bs + buf * kTileHalves + (wn * 64 + lrow) * kPadK + lk;
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            f16x8 a[4], b[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const f16x8*>(as + i * 32 * kPadK + kk);
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const f16x8*>(bs + j * 32 * kPadK + kk);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (s + 1 < steps) {
            ldsStore(buf ^ 1);
        }
        __syncthreads();
    }

    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<_Float16, _Float16>(A, B, C, lda, ldb, ldc, K, row0 + wm * 128, col0 + wn * 64, 128, 64, ACC);
        return;
    }
    // D layout of a 32x32 MFMA tile: lane l, register r holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t cBase = col0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                float* dst = C + row * ldc + cBase;
                const float v = acc[i][j][r];
                *dst = ACC ? *dst + v : v;
            }
        }
    }
}

/// Two-per-CU variant: a 128 x 256 workgroup tile of 4 waves (each 64 x 128 =
/// 2 x 4 MFMA tiles), K step 32, LDS tiles double buffered in 60 KiB, so
/// two workgroups share a CU and one's load waits overlap the other's MFMAs.
/// Global loads run two steps ahead in two register sets (the K loop is
/// unrolled by two so the sets are static; AHEAD2 = false loads one step
/// ahead in one set). A is staged as loaded ([m][k]);
/// B arrives as 4 (k) x 8 (n) blocks and is transposed in registers to
/// [n][k]; LDS rows are 40 halves (80 bytes), which keeps the 16-byte
/// operand reads conflict-free.
constexpr int kBM2 = 128, kBN2 = 256, kBK2 = 32, kPad2 = kBK2 + 8;
constexpr int kTileA2 = kBM2 * kPad2, kTileB2 = kBN2 * kPad2;
constexpr size_t kLdsGemm2 = 2 * (kTileA2 + kTileB2) * sizeof(_Float16);

__device__ __forceinline__ void xcdTile2(int tilesM, int tilesN, int& tm, int& tn) {
    // Consecutive ids go to different XCDs: give each XCD a contiguous block
    // of tile ids, row-major over (tm, tn) within the block.
    const int total = tilesM * tilesN;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    tm = id / tilesN;
    tn = id % tilesN;
}

template <bool ACC, bool AHEAD2>
__global__ __launch_bounds__(256, 2) void gemmF16Mfma2cu(const _Float16* __restrict__ A,
                                                         const _Float16* __restrict__ B,
                                                         float* __restrict__ C, int M, int N, int K,
                                                         int64_t lda, int64_t ldb, int64_t ldc, int skipZeroA) {
    extern __shared__ __align__(16) _Float16 lds[];
    _Float16* As = lds;                     // [2][128][40]
    _Float16* Bs = lds + 2 * kTileA2;       // [2][256][40]
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6, l32 = lane & 31, hl = lane >> 5;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    xcdTile2(M / kBM2, N / kBN2, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kBM2;
    const int64_t col0 = static_cast<int64_t>(tn) * kBN2;
    const int bk = t & 7;    // B block: k rows bk*4 .. +3
    const int bn = t >> 3;   // B block: n cols bn*8 .. +7
    u32x4 ra0[2], rb0[4], ra1[2], rb1[4];
    auto load = [&](int k0, u32x4(&ra)[2], u32x4(&rb)[4]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = j * 256 + t;   // 512 chunks: 128 rows x 4
            ra[j] = *reinterpret_cast<const u32x4*>(A + (row0 + (c >> 2)) * lda + k0 + (c & 3) * 8);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            rb[r] = *reinterpret_cast<const u32x4*>(B + static_cast<int64_t>(k0 + bk * 4 + r) * ldb + col0 + bn * 8);
        }
    };
    auto store = [&](int buf, const u32x4(&ra)[2], const u32x4(&rb)[4]) {
        _Float16* da = As + buf * kTileA2;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = j * 256 + t;
            *reinterpret_cast<u32x4*>(da + (c >> 2) * kPad2 + (c & 3) * 8) = ra[j];
        }
        _Float16* db = Bs + buf * kTileB2;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const int pp = n >> 1;
            const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
            uint32_t o0 = __builtin_amdgcn_perm(rb[1][pp], rb[0][pp], sel);
            uint32_t o1 = __builtin_amdgcn_perm(rb[3][pp], rb[2][pp], sel);
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            u32x2 o;
            o[0] = o0;
            o[1] = o1;
            *reinterpret_cast<u32x2*>(db + (bn * 8 + n) * kPad2 + bk * 4) = o;
        }
    };
    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
    }
    auto mfmaStep = [&](int buf) {
        const _Float16* as = As + buf * kTileA2 + (wm * 64 + l32) * kPad2 + hl * 8;
        const _Float16* bs = Bs + buf * kTileB2 + (wn * 128 + l32) * kPad2 + hl * 8;
#pragma unroll
        for (int kk = 0; kk < kBK2; kk += 16) {
            f16x8 a[2], b[4];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const f16x8*>(as + i * 32 * kPad2 + kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const f16x8*>(bs + j * 32 * kPad2 + kk);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    };
    // K / kBK2 is even (the launcher requires K % 64 == 0).
    const int steps = K / kBK2;
    load(0, ra0, rb0);
    store(0, ra0, rb0);
    if (AHEAD2) {
        load(kBK2, ra1, rb1);
        __syncthreads();
        for (int s = 0; s < steps; s += 2) {
            if (s + 2 < steps) load((s + 2) * kBK2, ra0, rb0);
            mfmaStep(0);
            store(1, ra1, rb1);
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
            if (s + 3 < steps) load((s + 3) * kBK2, ra1, rb1);
            mfmaStep(1);
            if (s + 2 < steps) store(0, ra0, rb0);
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        __syncthreads();
        for (int s = 0; s < steps; ++s) {
            if (s + 1 < steps) load((s + 1) * kBK2, ra0, rb0);
            mfmaStep(s & 1);
            if (s + 1 < steps) store((s + 1) & 1, ra0, rb0);
            __syncthreads();
        }
    }
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<_Float16, _Float16>(A, B, C, lda, ldb, ldc, K, row0 + wm * 64, col0 + wn * 128, 64, 128, ACC);
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t cBase = col0 + wn * 128 + j * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
                float* dst = C + row * ldc + cBase;
                const float v = acc[i][j][r];
                *dst = ACC ? *dst + v : v;
            }
        }
    }
}

/// 4-wave variant: the same 256x256x64 workgroup tile with each wave owning a
/// 128x128 quadrant (4x4 MFMA tiles, 256 accumulators in AGPRs), so every
/// kk step issues 8 LDS operand reads for 16 MFMAs. Thread t loads 8 A chunks
/// and one 8x8 B block per K step.
template <bool ACC>
__global__ __launch_bounds__(256) void gemmF16Mfma4w(const _Float16* __restrict__ A,
                                                     const _Float16* __restrict__ B,
                                                     float* __restrict__ C, int M, int N, int K,
                                                     int64_t lda, int64_t ldb, int64_t ldc,
                                                     int /*accumulate: template ACC*/, int skipZeroA) {
    extern __shared__ __align__(16) _Float16 lds[];
    _Float16* As = lds;
    _Float16* Bs = lds + 2 * kTileHalves;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave >> 1;   // 0..1
    const int wn = wave & 1;    // 0..1
    int tm, tn;
    xcdTile(M / kBM, N / kBN, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kBM;
    const int64_t col0 = static_cast<int64_t>(tn) * kBN;
    const int bk = t & 7;
    const int bn = t >> 3;
    u32x4 ra[8], rb[8];
    auto globalLoad = [&](int k0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = j * 256 + t;
            ra[j] = *reinterpret_cast<const u32x4*>(A + (row0 + (c >> 3)) * lda + k0 + (c & 7) * 8);
        }
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            rb[r] = *reinterpret_cast<const u32x4*>(B + static_cast<int64_t>(k0 + bk * 8 + r) * ldb + col0 + bn * 8);
        }
    };
    auto ldsStore = [&](int buf) {
        _Float16* da = As + buf * kTileHalves;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = j * 256 + t;
            *reinterpret_cast<u32x4*>(da + (c >> 3) * kPadK + (c & 7) * 8) = ra[j];
        }
        _Float16* db = Bs + buf * kTileHalves;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const int p = n >> 1;
            const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = __builtin_amdgcn_perm(rb[2 * j + 1][p], rb[2 * j][p], sel);
            *reinterpret_cast<u32x4*>(db + (bn * 8 + n) * kPadK + bk * 8) = o;
        }
    };
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
    }
    const int steps = K / kBK;
    globalLoad(0);
    ldsStore(0);
    __syncthreads();
    const int lrow = lane & 31;
    const int lk = (lane >> 5) * 8;
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        if (s + 1 < steps) globalLoad((s + 1) * kBK);
        const _Float16* as = As + buf * kTileHalves + (wm * 128 + lrow) * kPadK + lk;
        const _Float16* bs = Bs + buf * kTileHalves + (wn * 128 + lrow) * kPadK + lk;
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            f16x8 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const f16x8*>(as + i * 32 * kPadK + kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const f16x8*>(bs + j * 32 * kPadK + kk);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (s + 1 < steps) ldsStore(buf ^ 1);
        __syncthreads();
    }
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<_Float16, _Float16>(A, B, C, lda, ldb, ldc, K, row0 + wm * 128, col0 + wn * 128, 128, 128, ACC);
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t cBase = col0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                float* dst = C + row * ldc + cBase;
                const float v = acc[i][j][r];
                *dst = ACC ? *dst + v : v;
            }
        }
    }
}

/// 4-wave variant with A moved by the gfx950 direct global->LDS path
/// (global_load_lds_dwordx4): A never occupies VGPRs, which leaves room for
/// the 256 accumulators plus B's register staging without spills. A's LDS
/// tile is unpadded [256][64] with 16-byte chunks XOR-swizzled by
/// (row >> 1) & 7, so the 16 rows one quarter-wave reads hit 16 distinct
/// chunk slots. Each direct-load instruction writes 64 consecutive 16-byte
/// slots (lane i -> slot i); the lane chooses the global chunk that belongs
/// in that slot.
constexpr int kTileA = 256 * kBK;  // halves, unpadded

__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

template <bool ACC>
__global__ __launch_bounds__(256) void gemmF16Mfma4wDirect(const _Float16* __restrict__ A,
                                                           const _Float16* __restrict__ B,
                                                           float* __restrict__ C, int M, int N, int K,
                                                           int64_t lda, int64_t ldb, int64_t ldc,
                                                           int /*accumulate: template ACC*/, int skipZeroA) {
    extern __shared__ __align__(16) _Float16 lds[];
    _Float16* As = lds;                    // [2][256][64] swizzled
    _Float16* Bs = lds + 2 * kTileA;       // [2][256][kPadK]
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;
    int tm, tn;
    xcdTile(M / kBM, N / kBN, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kBM;
    const int64_t col0 = static_cast<int64_t>(tn) * kBN;
    const int bk = t & 7;
    const int bn = t >> 3;
    u32x4 rb[8];
    auto directA = [&](int k0, int buf) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int slot0 = (wave * 8 + j) * 64;          // first slot of this instruction
            const int q = slot0 + lane;
            const int row = q >> 3;
            const int c = (q & 7) ^ swz(row);               // logical chunk stored in slot q
            const _Float16* src = A + (row0 + row) * lda + k0 + c * 8;
            _Float16* dst = As + buf * kTileA + slot0 * 8;  // wave-uniform
            __builtin_amdgcn_global_load_lds(src, reinterpret_cast<__attribute__((address_space(3))) void*>(
                                                       reinterpret_cast<uintptr_t>(dst)),
                                             16, 0, 0);
        }
    };
    auto loadB = [&](int k0) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            rb[r] = *reinterpret_cast<const u32x4*>(B + static_cast<int64_t>(k0 + bk * 8 + r) * ldb + col0 + bn * 8);
        }
    };
    auto storeB = [&](int buf) {
        _Float16* db = Bs + buf * kTileHalves;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const int p = n >> 1;
            const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = __builtin_amdgcn_perm(rb[2 * j + 1][p], rb[2 * j][p], sel);
            *reinterpret_cast<u32x4*>(db + (bn * 8 + n) * kPadK + bk * 8) = o;
        }
    };
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
    }
    const int steps = K / kBK;
    directA(0, 0);
    loadB(0);
    storeB(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int lrow = lane & 31;
    const int lhalf = lane >> 5;
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        if (s + 1 < steps) {
            directA((s + 1) * kBK, buf ^ 1);
            loadB((s + 1) * kBK);
        }
        const _Float16* as = As + buf * kTileA;
        const _Float16* bs = Bs + buf * kTileHalves + (wn * 128 + lrow) * kPadK + lhalf * 8;
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            f16x8 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = wm * 128 + i * 32 + lrow;
                const int c = (kk >> 3) + lhalf;
                a[i] = *reinterpret_cast<const f16x8*>(as + row * kBK + ((c ^ swz(row)) * 8));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const f16x8*>(bs + j * 32 * kPadK + kk);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (s + 1 < steps) storeB(buf ^ 1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<_Float16, _Float16>(A, B, C, lda, ldb, ldc, K, row0 + wm * 128, col0 + wn * 128, 128, 128, ACC);
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t cBase = col0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                float* dst = C + row * ldc + cBase;
                const float v = acc[i][j][r];
                *dst = ACC ? *dst + v : v;
            }
        }
    }
}

/// Variant 3: variant 2's data movement with an explicit software pipeline
/// inside the K step. Operand fragments are double buffered in registers:
/// the 8 LDS reads for kk+1 are issued while the 16 MFMAs of kk run, and
/// sched_group_barrier pins the interleave (1 DS read per 2 MFMAs; the next
/// step's global loads spread over the first kk; the B transpose and its LDS
/// writes over the last kk), so the MFMA pipe never waits on LDS latency
/// except once after each barrier.
template <bool ACC>
__global__ __launch_bounds__(256) void gemmF16Mfma4wPipe(const _Float16* __restrict__ A,
                                                         const _Float16* __restrict__ B,
                                                         float* __restrict__ C, int M, int N, int K,
                                                         int64_t lda, int64_t ldb, int64_t ldc, int skipZeroA) {
    extern __shared__ __align__(16) _Float16 lds[];
    _Float16* As = lds;
    _Float16* Bs = lds + 2 * kTileA;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;
    int tm, tn;
    xcdTile(M / kBM, N / kBN, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kBM;
    const int64_t col0 = static_cast<int64_t>(tn) * kBN;
    const int bk = t & 7;
    const int bn = t >> 3;
    const int lrow = lane & 31;
    const int lhalf = lane >> 5;
    u32x4 rb[8];
    auto directA = [&](int k0, int buf) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int slot0 = (wave * 8 + j) * 64;
            const int q = slot0 + lane;
            const int row = q >> 3;
            const int c = (q & 7) ^ swz(row);
            const _Float16* src = A + (row0 + row) * lda + k0 + c * 8;
            _Float16* dst = As + buf * kTileA + slot0 * 8;
            __builtin_amdgcn_global_load_lds(src, reinterpret_cast<__attribute__((address_space(3))) void*>(
                                                       reinterpret_cast<uintptr_t>(dst)),
                                             16, 0, 0);
        }
    };
    auto loadB = [&](int k0) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            rb[r] = *reinterpret_cast<const u32x4*>(B + static_cast<int64_t>(k0 + bk * 8 + r) * ldb + col0 + bn * 8);
        }
    };
    auto storeB = [&](int buf) {
        _Float16* db = Bs + buf * kTileHalves;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const int p = n >> 1;
            const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = __builtin_amdgcn_perm(rb[2 * j + 1][p], rb[2 * j][p], sel);
            *reinterpret_cast<u32x4*>(db + (bn * 8 + n) * kPadK + bk * 8) = o;
        }
    };
    f16x8 fa[2][4], fb[2][4];
    auto readFrags = [&](int buf, int kk, int slot) {
        const _Float16* as = As + buf * kTileA;
        const _Float16* bs = Bs + buf * kTileHalves + (wn * 128 + lrow) * kPadK + lhalf * 8 + kk;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = wm * 128 + i * 32 + lrow;
            const int c = (kk >> 3) + lhalf;
            fa[slot][i] = *reinterpret_cast<const f16x8*>(as + row * kBK + ((c ^ swz(row)) * 8));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) fb[slot][j] = *reinterpret_cast<const f16x8*>(bs + j * 32 * kPadK);
    };
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
    }
    auto mfmas = [&](int slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[slot][i], fb[slot][j], acc[i][j], 0, 0, 0);
            }
        }
    };
    const int steps = K / kBK;
    directA(0, 0);
    loadB(0);
    storeB(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        // Branch-free step body (one scheduling region): the last step
        // re-loads its own, in-bounds K slice into the idle buffer.
        const int kNext = (s + 1 < steps ? s + 1 : s) * kBK;
        readFrags(buf, 0, 0);
        directA(kNext, buf ^ 1);
        loadB(kNext);
        // kk = 0: next fragments + the next step's global loads.
        readFrags(buf, 16, 1);
        mfmas(0);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // 1 DS read
            __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);   // 2 VMEM reads
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // 2 MFMA
        }
        readFrags(buf, 32, 0);
        mfmas(1);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        readFrags(buf, 48, 1);
        mfmas(0);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        mfmas(1);
        storeB(buf ^ 1);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // 4 VALU (transpose)
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // 1 DS write
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // 2 MFMA
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<_Float16, _Float16>(A, B, C, lda, ldb, ldc, K, row0 + wm * 128, col0 + wn * 128, 128, 128, ACC);
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t cBase = col0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                float* dst = C + row * ldc + cBase;
                const float v = acc[i][j][r];
                *dst = ACC ? *dst + v : v;
            }
        }
    }
}

/// Variant 7: both operands moved global -> LDS by the gfx950 direct path
/// (global_load_lds_dwordx4, no VGPR staging) into a 4-deep ring of K steps
/// of 32; B is kept as loaded ([k][n]) and read with ds_read_b64_tr_b16,
/// which hands each lane 4 consecutive k of one column, i.e. the MFMA B
/// operand without a register transpose. 4 waves (2 x 2), each owning a
/// 128 x 128 quadrant (4 x 4 MFMA tiles, 256 accumulators). The fragments of
/// the next 16-deep sub-step are read while the current one's 16 MFMAs run
/// (one LDS read per MFMA). One barrier per K step certifies the next stage;
/// every step issues exactly one stage (past the end a harmless reload into
/// a slot nothing reads), so the wait before the barrier is a constant
/// vmcnt. The direct loads are inline asm: the kernel accounts for them
/// itself, so the compiler adds no conservative waits on them.
/// LDS swizzles: A rows are 64 bytes (4 chunks), chunk c of row r sits at
/// c ^ ((r >> 2) & 3); B rows are 512 bytes, chunk c of k-row r sits at
/// c ^ ((r & 3) * 4). Both measured conflict-free (SQ_LDS_BANK_CONFLICT 0).
constexpr int kDmaBK = 32, kDmaStages = 4;
constexpr int kDmaA = 256 * kDmaBK;                   // halves per A stage
constexpr int kDmaStage = 2 * kDmaA;                  // A then B
constexpr size_t kLdsDma = static_cast<size_t>(kDmaStages) * kDmaStage * sizeof(_Float16);   // 128 KiB

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));

__device__ __forceinline__ uint32_t ldsOffset(const void* p) {
    // Generic pointers into LDS carry the LDS offset in their low 32 bits.
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

/// 16 bytes per lane from `src` to LDS `dst` + 16 * lane; `dst` is the same
/// for the whole wave and goes through M0. M0 is a reserved register: naming
/// it as a clobber only draws a warning that reserved registers are not
/// preserved, so it is left out. The asm sets M0 itself right before the
/// load, and in the kernels that use these loads every M0 write comes from
/// these asm statements (the compiled code holds no other value in M0).
__device__ __forceinline__ void dmaLoad16(const _Float16* src, const _Float16* dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(ldsOffset(dst));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory");
}

struct DmaFrag {
    f16x8 a[4];
    f16x4 b[4][2];
};

template <bool ACC>
__global__ __launch_bounds__(256, 1) void gemmF16Dma(const _Float16* __restrict__ A,
                                                     const _Float16* __restrict__ B,
                                                     float* __restrict__ C, int M, int N, int K,
                                                     int64_t lda, int64_t ldb, int64_t ldc, int skipZeroA) {
    extern __shared__ __align__(16) _Float16 lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    xcdTile(M / kBM, N / kBN, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kBM;
    const int64_t col0 = static_cast<int64_t>(tn) * kBN;
    const int steps = K / kDmaBK;

    // Stage `slot` receives K step min(slot, steps - 1) in ring slot
    // slot % kDmaStages. Wave w issues A instructions 4w..4w+3 (16 rows
    // each) and B instructions 4w..4w+3 (2 k-rows each).
    auto issue = [&](int slot) {
        const int k0 = min(slot, steps - 1) * kDmaBK;
        const _Float16* st = lds + (slot % kDmaStages) * kDmaStage;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ins = wave * 4 + j;
            const int q = ins * 64 + lane;
            const int row = q >> 2;
            const int c = (q & 3) ^ ((row >> 2) & 3);
            dmaLoad16(A + (row0 + row) * lda + k0 + c * 8, st + ins * 512);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ins = wave * 4 + j;
            const int q = ins * 64 + lane;
            const int krow = q >> 5;
            const int c = (q & 31) ^ ((krow & 3) * 4);
            dmaLoad16(B + static_cast<int64_t>(k0 + krow) * ldb + col0 + c * 8, st + kDmaA + ins * 512);
        }
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
    }
#pragma unroll
    for (int s = 0; s < kDmaStages - 1; ++s) issue(s);

    const int l32 = lane & 31, hl = lane >> 5;
    const int g = lane >> 4, sl = lane & 15;
    // Lane byte offsets inside a stage. A: per sub-step kk (tile i adds 32
    // rows = 2048 bytes). B: per (kk, j, h) for the two 4-deep halves of the
    // transposed read (lanes of group g read k-rows 8 * (g >> 1) + sl / 4).
    uint32_t offA[2], offB[2][4][2];
    {
        const int row = wm * 128 + l32;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) offA[kk] = 2u * (row * kDmaBK + (((kk * 2 + hl) ^ ((row >> 2) & 3)) * 8));
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int krow = kk * 16 + 8 * (g >> 1) + (sl >> 2) + 4 * h;
                    const int col = wn * 128 + j * 32 + 16 * (g & 1) + 4 * (sl & 3);
                    offB[kk][j][h] = 2u * (kDmaA + krow * 256 + (((col >> 3) ^ ((krow & 3) * 4)) * 8) + (col & 7));
                }
            }
        }
    }
    const uint32_t ldsBase = ldsOffset(lds);
    // Read r of a sub-step: r 0..3 the A tiles, r 4..11 the B halves (j, h).
    auto readOne = [&](DmaFrag& f, uint32_t base, int kk, int r) {
        if (r < 4) {
            f.a[r] = *reinterpret_cast<const __attribute__((address_space(3))) f16x8*>(base + offA[kk] + 2048u * r);
        } else {
            const int j = (r - 4) >> 1, h = (r - 4) & 1;
            const fp16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                reinterpret_cast<__attribute__((address_space(3))) fp16x4*>(base + offB[kk][j][h]));
            f.b[j][h] = __builtin_bit_cast(f16x4, v);
        }
    };
    auto mfma = [&](const DmaFrag& f, int idx) {
        const int i = idx >> 2, j = idx & 3;
        const f16x8 bb = __builtin_shufflevector(f.b[j][0], f.b[j][1], 0, 1, 2, 3, 4, 5, 6, 7);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], bb, acc[i][j], 0, 0, 0);
    };
    // 16 MFMAs of `cur` with the 12 reads of the next sub-step between them.
    auto subStep = [&](DmaFrag& cur, DmaFrag& nxt, uint32_t nbase, int nkk) {
#pragma unroll
        for (int idx = 0; idx < 16; ++idx) {
            mfma(cur, idx);
            if (idx < 12) readOne(nxt, nbase, nkk, idx);
        }
#pragma unroll
        for (int idx = 0; idx < 12; ++idx) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };

    DmaFrag x, y;
    // Stage 0 landed (stages 1 and 2, 8 direct loads each per wave, may be
    // in flight).
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
#pragma unroll
    for (int r = 0; r < 12; ++r) readOne(x, ldsBase, 0, r);
    for (int s = 0; s < steps; ++s) {
        const uint32_t cb = ldsBase + 2u * static_cast<uint32_t>((s % kDmaStages) * kDmaStage);
        subStep(x, y, cb, 1);   // sub-step (s, 0); reads (s, 1)
        // Stage s + 1 landed (one later stage, 8 direct loads per wave, may be
        // in flight); after the barrier every wave is past step s - 1, so its
        // slot can be refilled.
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        asm volatile("s_barrier" ::: "memory");
        issue(s + kDmaStages - 1);
        const uint32_t nb = ldsBase + 2u * static_cast<uint32_t>(((s + 1) % kDmaStages) * kDmaStage);
        subStep(y, x, nb, 0);   // sub-step (s, 1); reads (s + 1, 0)
    }
    // No direct load may still be writing LDS when the workgroup ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<_Float16, _Float16>(A, B, C, lda, ldb, ldc, K, row0 + wm * 128, col0 + wn * 128, 128, 128, ACC);
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t cBase = col0 + wn * 128 + j * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
                float* dst = C + row * ldc + cBase;
                const float v = acc[i][j][r];
                *dst = ACC ? *dst + v : v;
            }
        }
    }
}

/// Variant 8: variant 7's data movement (the same 4-deep direct-to-LDS ring
/// of K steps of 32, the same swizzles and transposed B reads) with 8 waves
/// (2 per SIMD, 2 (M) x 4 (N)), each owning 128 x 64, and
/// v_mfma_f32_16x16x32_f16 with the operands swapped: each 16 x 16 tile is
/// D = B^T A^T, so a lane holds 4 consecutive columns of one row of C and
/// stores them with one 16-byte write. The 32 tiles of a wave (8 x 4) keep
/// their 128 accumulators in ordinary registers. Under this chip's power
/// limit the smaller MFMA sustains more work per joule (a register-only loop
/// runs 12% faster with it than with 32x32x16). Each K step is two groups of
/// 16 MFMAs (m-tiles 0-3, then 4-7): the first group's MFMAs overlap the
/// reads of the second group's A fragments; the barrier that certifies the
/// next stage sits between the groups, and the second group overlaps the
/// reads of the next step's first group (B fragments double buffered).
/// Every output element takes its products in the same k order as variant
/// 7, and the results match it bit for bit. Needs K a multiple of 64.
template <bool ACC>
__global__ __launch_bounds__(512, 1) void gemmF16Dma8(const _Float16* __restrict__ A,
                                                      const _Float16* __restrict__ B,
                                                      float* __restrict__ C, int M, int N, int K,
                                                      int64_t lda, int64_t ldb, int64_t ldc, int skipZeroA) {
    extern __shared__ __align__(16) _Float16 lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    int tm, tn;
    xcdTile(M / kBM, N / kBN, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kBM;
    const int64_t col0 = static_cast<int64_t>(tn) * kBN;
    const int steps = K / kDmaBK;

    // Stage `slot` receives K step min(slot, steps - 1) in ring slot
    // slot % kDmaStages. Wave w issues A instructions 2w, 2w + 1 (16 rows
    // each) and B instructions 2w, 2w + 1 (2 k-rows each).
    auto issue = [&](int slot) {
        const int k0 = min(slot, steps - 1) * kDmaBK;
        const _Float16* st = lds + (slot % kDmaStages) * kDmaStage;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ins = wave * 2 + j;
            const int q = ins * 64 + lane;
            const int row = q >> 2;
            const int c = (q & 3) ^ ((row >> 2) & 3);
            dmaLoad16(A + (row0 + row) * lda + k0 + c * 8, st + ins * 512);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ins = wave * 2 + j;
            const int q = ins * 64 + lane;
            const int krow = q >> 5;
            const int c = (q & 31) ^ ((krow & 3) * 4);
            dmaLoad16(B + static_cast<int64_t>(k0 + krow) * ldb + col0 + c * 8, st + kDmaA + ins * 512);
        }
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
        }
    }
#pragma unroll
    for (int s = 0; s < kDmaStages - 1; ++s) issue(s);

    const int l16 = lane & 15, g = lane >> 4;
    // The MFMA's B operand (A^T): row wm * 128 + 16 mt + l16 of A, chunk g
    // (k 8g .. 8g + 7) at its swizzled slot; tile mt adds 1024 bytes.
    uint32_t offA;
    {
        const int row = wm * 128 + l16;
        offA = 2u * (row * kDmaBK + ((g ^ ((row >> 2) & 3)) * 8));
    }
    // The MFMA's A operand (B^T): column wn * 64 + 16 nt + l16 of B, k 8g ..
    // 8g + 7 by two transposed reads (h = 0, 1); lane (g, l16) points at
    // k-row 8g + 4h + l16 / 4, columns 4 (l16 % 4) .. + 3 of the tile.
    uint32_t offB[4][2];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int krow = 8 * g + 4 * h + (l16 >> 2);
            const int col = wn * 64 + nt * 16 + 4 * (l16 & 3);
            offB[nt][h] = 2u * (kDmaA + krow * 256 + (((col >> 3) ^ ((krow & 3) * 4)) * 8) + (col & 7));
        }
    }
    const uint32_t ldsBase = ldsOffset(lds);
    auto readA = [&](f16x8& f, uint32_t base, int mt) {
        f = *reinterpret_cast<const __attribute__((address_space(3))) f16x8*>(base + offA + 1024u * mt);
    };
    auto readB = [&](f16x8& f, uint32_t base, int nt) {
        const fp16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            reinterpret_cast<__attribute__((address_space(3))) fp16x4*>(base + offB[nt][0]));
        const fp16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            reinterpret_cast<__attribute__((address_space(3))) fp16x4*>(base + offB[nt][1]));
        f = __builtin_shufflevector(__builtin_bit_cast(f16x4, v0), __builtin_bit_cast(f16x4, v1), 0, 1, 2, 3, 4, 5,
                                    6, 7);
    };
    f16x8 aLo[4], aHi[4], bX[4], bY[4];
    // 16 MFMAs: m-tiles mt0 .. mt0 + 3 against the 4 n-tiles.
    auto group = [&](const f16x8 (&a)[4], const f16x8 (&b)[4], int mt0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[mt0 + i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[j], a[i], acc[mt0 + i][j], 0, 0, 0);
            }
        }
    };
    // Stage 0 landed (stages 1 and 2, 4 direct loads each per wave, may be
    // in flight).
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i) readA(aLo[i], ldsBase, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) readB(bX[j], ldsBase, j);
    auto step = [&](int s, f16x8 (&bCur)[4], f16x8 (&bNxt)[4]) {
        const uint32_t cb = ldsBase + 2u * static_cast<uint32_t>((s % kDmaStages) * kDmaStage);
        group(aLo, bCur, 0);                          // m-tiles 0-3 of step s; reads m-tiles 4-7
#pragma unroll
        for (int i = 0; i < 4; ++i) readA(aHi[i], cb, 4 + i);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            if (i < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        // Stage s + 1 landed (one later stage may be in flight); after the
        // barrier every wave is past step s - 1, so its slot can be refilled.
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        asm volatile("s_barrier" ::: "memory");
        issue(s + kDmaStages - 1);
        const uint32_t nb = ldsBase + 2u * static_cast<uint32_t>(((s + 1) % kDmaStages) * kDmaStage);
        group(aHi, bCur, 4);                          // m-tiles 4-7 of step s; reads step s + 1's first group
#pragma unroll
        for (int i = 0; i < 4; ++i) readA(aLo[i], nb, i);
#pragma unroll
        for (int j = 0; j < 4; ++j) readB(bNxt[j], nb, j);
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };
    for (int s = 0; s < steps; s += 2) {              // steps is even (K % 64 == 0)
        step(s, bX, bY);
        step(s + 1, bY, bX);
    }
    // No direct load may still be writing LDS when the workgroup ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<_Float16, _Float16>(A, B, C, lda, ldb, ldc, K, row0 + wm * 128, col0 + wn * 64, 128, 64, ACC);
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t row = row0 + wm * 128 + i * 16 + l16;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4* dst = reinterpret_cast<f32x4*>(C + row * ldc + col0 + wn * 64 + j * 16 + 4 * g);
            f32x4 v = acc[i][j];
            if (ACC) v += *dst;
            *dst = v;
        }
    }
}

/// Direct load through a scalar base: lane bytes `voff` past `sbase` into LDS
/// at M0 + 16 * lane. The K advance lives in `sbase` (scalar adds), so the
/// per-lane address costs no vector instruction per step.
/// M0 is handled as in dmaLoad16.
__device__ __forceinline__ void dmaLoad16s(const void* sbase, uint32_t voff, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(m0) : "memory");
}

/// Variant 8 (K a multiple of 64): the same tiles, ring, swizzles and
/// per-accumulator MFMAs as gemmF16Dma8 (results identical bit for bit), with
/// no per-step vector address arithmetic and a fixed instruction order.
/// * Vector instructions take issue cycles from the MFMAs of the wave sharing
///   the SIMD (measured on gfx950: 32 v_add_u32 per 32 MFMAs cost 9% of the
///   MFMA rate, 16 v_readfirstlane 18%). gemmF16Dma8 spends about 40 per K
///   step on addresses: 64-bit adds, multiplies by ldb and a readfirstlane
///   per direct load. Here the direct loads take a scalar base plus a fixed
///   32-bit lane offset and M0 comes from scalar registers; the loop is
///   unrolled over the 4 ring slots so that every LDS fragment read is a
///   base register plus an immediate offset (two bases per operand, since
///   DS offsets hold 16 bits).
/// * The compiler does not keep the interleave that sched_group_barrier asks
///   for across the unrolled steps: it hoists the next step's first MFMAs up
///   to the reads that feed them and then waits for those reads every one or
///   two MFMAs. Scheduling fences after each MFMA pin the order, with the
///   memory instructions spread out rather than bunched: the next m-tiles'
///   A reads after every other MFMA of group 1's first half, the next step's
///   fragments after every other MFMA of group 2 in order of first use, and
///   the four direct loads of the stage after every fourth MFMA of group 2
///   from the third (3-4% faster than the same instructions bunched at the
///   start of each group, with identical results).
/// * Within a group the MFMAs walk the 4 x 4 tiles row by row in a snake
///   (n ascending on even m-tiles, descending on odd ones), so every two
///   consecutive MFMAs share an operand register (0.8% faster than plain
///   row order, identical results).
/// Needs lda < 2^23 and ldb < 2^25 (32-bit lane offsets).
template <bool ACC>
__global__ __launch_bounds__(512, 1) void gemmF16Dma8s(const _Float16* __restrict__ A,
                                                       const _Float16* __restrict__ B,
                                                       float* __restrict__ C, int M, int N, int K,
                                                       int64_t lda, int64_t ldb, int64_t ldc,
                                                       int skipZeroA) {
    extern __shared__ __align__(16) _Float16 lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int wm = wave >> 2, wn = wave & 3;
    int tm, tn;
    xcdTile(M / kBM, N / kBN, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kBM;
    const int64_t col0 = static_cast<int64_t>(tn) * kBN;
    const int steps = K / kDmaBK;

    // Wave w's direct loads are A instructions 2w, 2w + 1 (16 rows each) and
    // B instructions 2w, 2w + 1 (2 k-rows each) of every stage, as in
    // gemmF16Dma8: lane byte offsets from the tile's A rows / B columns.
    uint32_t gA[2], gB[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int q = (wave * 2 + j) * 64 + lane;
        const int row = q >> 2;
        const int c = (q & 3) ^ ((row >> 2) & 3);
        gA[j] = static_cast<uint32_t>((row * lda + c * 8) * 2);
        const int krow = q >> 5;
        const int cb = (q & 31) ^ ((krow & 3) * 4);
        gB[j] = static_cast<uint32_t>((krow * ldb + cb * 8) * 2);
    }
    const char* aTile = reinterpret_cast<const char*>(A + row0 * lda);
    const char* bTile = reinterpret_cast<const char*>(B + col0);
    const uint32_t ldsS = __builtin_amdgcn_readfirstlane(ldsOffset(lds));
    const uint32_t m0Wave = ldsS + static_cast<uint32_t>(wave) * 2048u;
    // Direct load j (A 0, A 1, B 0, B 1) of stage t (K step min(t, steps - 1))
    // into ring slot `slot` = t % 4.
    auto issueOne = [&](int t, const int slot, const int j) {
        const int64_t k0 = static_cast<int64_t>(min(t, steps - 1)) * kDmaBK;
        const char* a = aTile + k0 * 2;
        const char* b = bTile + k0 * ldb * 2;
        const uint32_t m = m0Wave + static_cast<uint32_t>(slot) * (kDmaStage * 2u);
        if (j == 0) dmaLoad16s(a, gA[0], m);
        if (j == 1) dmaLoad16s(a, gA[1], m + 1024u);
        if (j == 2) dmaLoad16s(b, gB[0], m + kDmaA * 2u);
        if (j == 3) dmaLoad16s(b, gB[1], m + kDmaA * 2u + 1024u);
    };
    auto issue = [&](int t, const int slot) {
#pragma unroll
        for (int j = 0; j < 4; ++j) issueOne(t, slot, j);
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    issue(0, 0);
    issue(1, 1);
    issue(2, 2);

    // Fragment bases: slots 0 and 1 from vA0 / vB0, slots 2 and 3 from the
    // bases 64 KiB up; the slot's remaining 0 or 32 KiB, the m-tile (1 KiB)
    // and the second transposed half (4 k-rows, 2 KiB) are immediates.
    const int l16 = lane & 15, g = lane >> 4;
    uint32_t vA0;
    {
        const int row = wm * 128 + l16;
        vA0 = ldsS + 2u * (row * kDmaBK + ((g ^ ((row >> 2) & 3)) * 8));
    }
    uint32_t vB0[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const int krow = 8 * g + (l16 >> 2);
        const int col = wn * 64 + nt * 16 + 4 * (l16 & 3);
        vB0[nt] = ldsS + 2u * (kDmaA + krow * 256 + (((col >> 3) ^ ((krow & 3) * 4)) * 8) + (col & 7));
    }
    const uint32_t vA2 = vA0 + 65536u;
    uint32_t vB2[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) vB2[nt] = vB0[nt] + 65536u;
    auto readA = [&](f16x8& f, const int slot, int mt) {
        const uint32_t addr = (slot < 2 ? vA0 : vA2) + static_cast<uint32_t>((slot & 1) * kDmaStage * 2 + 1024 * mt);
        f = *reinterpret_cast<const __attribute__((address_space(3))) f16x8*>(addr);
    };
    auto readB = [&](f16x8& f, const int slot, int nt) {
        const uint32_t base = (slot < 2 ? vB0[nt] : vB2[nt]) + static_cast<uint32_t>((slot & 1) * kDmaStage * 2);
        const fp16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            reinterpret_cast<__attribute__((address_space(3))) fp16x4*>(base));
        const fp16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            reinterpret_cast<__attribute__((address_space(3))) fp16x4*>(base + 2048u));
        f = __builtin_shufflevector(__builtin_bit_cast(f16x4, v0), __builtin_bit_cast(f16x4, v1), 0, 1, 2, 3, 4, 5,
                                    6, 7);
    };
    f16x8 aLo[4], aHi[4], bX[4], bY[4];
    // Stage 0 landed (stages 1 and 2, 4 direct loads each per wave, may be in
    // flight).
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i) readA(aLo[i], 0, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) readB(bX[j], 0, j);
    auto mfma = [&](const f16x8& a, const f16x8& b, f32x4& c) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a, c, 0, 0, 0);
    };
    // K step s in ring slot q = s % 4.
    auto step = [&](int s, const int q, f16x8 (&bCur)[4], f16x8 (&bNxt)[4]) {
        const int qn = (q + 1) & 3;
        // Group 1: m-tiles 0-3; the A fragments of m-tiles 4-7 are read
        // behind MFMAs 0, 2, 4 and 6.
#pragma unroll
        for (int idx = 0; idx < 16; ++idx) {
            const int mi = idx >> 2, ni = (mi & 1) ? 3 - (idx & 3) : (idx & 3);
            mfma(aLo[mi], bCur[ni], acc[mi][ni]);
            if (idx < 8 && (idx & 1) == 0) readA(aHi[idx >> 1], q, 4 + (idx >> 1));
            __builtin_amdgcn_sched_barrier(0);
        }
        // Stage s + 1 landed (one later stage may be in flight); after the
        // barrier every wave is past step s - 1, so its slot can be refilled.
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // Group 2: m-tiles 4-7; step s + 1's fragments read behind the even
        // MFMAs in order of first use (B 0, A 0, B 1-3, A 1-3), and stage
        // s + 3's direct loads into slot (s - 1) % 4 behind MFMAs 2, 6, 10, 14.
#pragma unroll
        for (int idx = 0; idx < 16; ++idx) {
            const int mi = idx >> 2, ni = (mi & 1) ? 3 - (idx & 3) : (idx & 3);
            mfma(aHi[mi], bCur[ni], acc[4 + mi][ni]);
            if (idx == 0) readB(bNxt[0], qn, 0);
            if (idx == 2) readA(aLo[0], qn, 0);
            if (idx >= 4 && idx <= 8 && (idx & 1) == 0) readB(bNxt[(idx - 2) >> 1], qn, (idx - 2) >> 1);
            if (idx >= 10 && (idx & 1) == 0) readA(aLo[(idx - 8) >> 1], qn, (idx - 8) >> 1);
            if ((idx & 3) == 2) issueOne(s + kDmaStages - 1, (q + 3) & 3, idx >> 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    int s = 0;
    for (; s + 4 <= steps; s += 4) {
        step(s, 0, bX, bY);
        step(s + 1, 1, bY, bX);
        step(s + 2, 2, bX, bY);
        step(s + 3, 3, bY, bX);
    }
    if (s < steps) {   // K % 128 == 64: two more steps, in slots 0 and 1
        step(s, 0, bX, bY);
        step(s + 1, 1, bY, bX);
    }
    // No direct load may still be writing LDS when the workgroup ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<_Float16, _Float16>(A, B, C, lda, ldb, ldc, K, row0 + wm * 128, col0 + wn * 64, 128, 64, ACC);
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t row = row0 + wm * 128 + i * 16 + l16;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4* dst = reinterpret_cast<f32x4*>(C + row * ldc + col0 + wn * 64 + j * 16 + 4 * g);
            f32x4 v = acc[i][j];
            if (ACC) v += *dst;
            *dst = v;
        }
    }
}

// ---------------------------------------------------------------- f32 ----
constexpr int kFM = 64, kFN = 64, kFK = 32;
constexpr int kFDepth = 2;   // K steps of global loads in flight ahead of the MFMAs

/// f32 form 1: 64x64 output tile per workgroup of 4 waves (2 x 2 of 32x32),
/// K steps of 32 through double-buffered LDS, v_mfma_f32_32x32x2f32 with k
/// ascending.
/// Global loads run kFDepth steps ahead in registers (slot t % kFDepth holds
/// step t); A is stored transposed ([k][m]) for the MFMA's A operand, and its
/// load mapping gives each wave 16 rows x 4 k-chunks, so every transposed LDS
/// write of a wave hits 64 distinct banks. At 1024^3 on gfx950: 25-26 us,
/// against 29-31 us with one step in flight and the row-major mapping
/// (4-way write conflicts).
template <bool ACC>
__global__ __launch_bounds__(256) void gemmF32Mfma(const float* __restrict__ A,
                                                   const float* __restrict__ B,
                                                   float* __restrict__ C, int /*M: the grid covers it*/, int N,
                                                   int K, int64_t lda, int64_t ldb, int64_t ldc,
                                                   int /*accumulate: template ACC*/, int skipZeroA) {
    __shared__ float At[2][kFK][kFM + 4];   // transposed: [k][m]
    __shared__ float Bs[2][kFK][kFN + 4];   // as loaded: [k][n]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;   // 2x2 waves, 32x32 each
    const int tilesN = N / kFN;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x / tilesN) * kFM;
    const int64_t col0 = static_cast<int64_t>(blockIdx.x % tilesN) * kFN;

    // A tile 64x32 floats = 512 float4 and B tile 32x64 = 512 float4: 2 of
    // each per thread. Item c of A: wave-slice q = c / 64 covers rows
    // 16 (q / 2) .. +15 and k-chunks 4 (q % 2) .. +3.
    auto aItem = [&](int c, int& r, int& ch) {
        const int q = c >> 6, ln = c & 63;
        r = (q >> 1) * 16 + (ln & 15);
        ch = (q & 1) * 4 + (ln >> 4);
    };
    f32x4 ra[kFDepth][2], rb[kFDepth][2];
    auto globalLoad = [&](int k0, f32x4 (&xa)[2], f32x4 (&xb)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = j * 256 + tid;
            int r, ch;
            aItem(c, r, ch);
            xa[j] = *reinterpret_cast<const f32x4*>(A + (row0 + r) * lda + k0 + ch * 4);
            const int kr = c >> 4, nc = c & 15;     // B: 32 rows x 16 chunks
            xb[j] = *reinterpret_cast<const f32x4*>(B + static_cast<int64_t>(k0 + kr) * ldb + col0 + nc * 4);
        }
    };
    auto ldsStore = [&](int buf, const f32x4 (&xa)[2], const f32x4 (&xb)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = j * 256 + tid;
            int r, ch;
            aItem(c, r, ch);
#pragma unroll
            for (int e = 0; e < 4; ++e) At[buf][ch * 4 + e][r] = xa[j][e];
            const int kr = c >> 4, nc = c & 15;
            *reinterpret_cast<f32x4*>(&Bs[buf][kr][nc * 4]) = xb[j];
        }
    };
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const int steps = K / kFK;
#pragma unroll
    for (int d = 0; d < kFDepth; ++d) {
        if (d < steps) globalLoad(d * kFK, ra[d], rb[d]);
    }
    ldsStore(0, ra[0], rb[0]);
    __syncthreads();
    const int lcol = lane & 31;
    const int lk = lane >> 5;
    for (int s0 = 0; s0 < steps; s0 += kFDepth) {
#pragma unroll
        for (int d = 0; d < kFDepth; ++d) {
            const int s = s0 + d;
            if (s < steps) {
                const int buf = s & 1;
                // Slot d held step s, already in LDS: refill it with s + kFDepth.
                if (s + kFDepth < steps) globalLoad((s + kFDepth) * kFK, ra[d], rb[d]);
#pragma unroll
                for (int kk = 0; kk < kFK; kk += 2) {
                    const float a = At[buf][kk + lk][wm * 32 + lcol];
                    const float b = Bs[buf][kk + lk][wn * 32 + lcol];
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
                }
                if (s + 1 < steps) ldsStore(buf ^ 1, ra[(d + 1) % kFDepth], rb[(d + 1) % kFDepth]);
                __syncthreads();
            }
        }
    }
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<float, float>(A, B, C, lda, ldb, ldc, K, row0 + wm * 32, col0 + wn * 32, 32, 32, ACC);
        return;
    }
    const int64_t cBase = col0 + wn * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t row = row0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        float* dst = C + row * ldc + cBase;
        *dst = ACC ? *dst + acc[r] : acc[r];
    }
}

/// f32 form 0: both 64x64 tiles move global -> LDS by the direct path
/// (global_load_lds_dwordx4, no register staging and no LDS writes) into a
/// 4-deep ring of K steps of 64 (32 KiB per stage). 8 waves: waves q and
/// q + 4 own the same 32x32 tile (2 x 2 quadrants) on v_mfma_f32_32x32x2_f32
/// and take the two halves of every K step, so each SIMD runs two
/// independent accumulator chains. Within a step the k order is permuted:
/// MFMA t takes k = t from lanes 0-31 and k = 32 + t from lanes 32-63; wave
/// half h takes t = 16h .. 16h + 15. The A operand of 4 consecutive MFMAs is
/// then one 16-byte read of a row of A (16-byte chunk c of row m sits at
/// c ^ (m & 15): the 16 rows a quarter-wave reads hit 16 distinct slots),
/// and the B operand a 4-byte read of 32 consecutive columns. One barrier
/// per K step; every step issues exactly one stage (past the end a harmless
/// reload into a slot nothing reads), so the wait before the barrier is a
/// constant vmcnt. At the end the second half's sums reach the first half's
/// waves through LDS and each output is half 0 + half 1, in that order.
/// Needs K a multiple of 64. Each output's sum runs over k in a different
/// order from form 1's k ascending, within the f32 tolerance.
constexpr int kQK = 64, kQStages = 4;
constexpr int kQA = kFM * kQK;                        // floats per A stage (64 rows x 64 k)
constexpr int kQStage = 2 * kQA;                      // A, then B (64 k x 64 n)
constexpr size_t kLdsF32Dma = static_cast<size_t>(kQStages) * kQStage * sizeof(float);   // 128 KiB

template <bool ACC>
__global__ __launch_bounds__(512, 1) void gemmF32Dma(const float* __restrict__ A, const float* __restrict__ B,
                                                     float* __restrict__ C, int N, int K, int64_t lda,
                                                     int64_t ldb, int64_t ldc, int skipZeroA) {
    extern __shared__ __align__(16) float ldsF[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int quad = wave & 3, h = wave >> 2;   // output quadrant, K-step half
    const int wm = quad >> 1, wn = quad & 1;
    const int tilesN = N / kFN;
    // XCD-blocked map: at 1024^2 each XCD's 32 tiles form a 4 x 8 block, so
    // its L2 holds 4 A and 8 B panels (3 MiB) instead of 16 A panels; the
    // bytes fetched per launch drop by a third (FETCH_SIZE 18470 -> 12330 KiB).
    int tm, tn;
    xcdTile(static_cast<int>(gridDim.x) / tilesN, tilesN, tm, tn);
    const int64_t row0 = static_cast<int64_t>(tm) * kFM;
    const int64_t col0 = static_cast<int64_t>(tn) * kFN;
    const int steps = K / kQK;
    // Stage `slot` receives K step min(slot, steps - 1) in ring slot
    // slot % kQStages. A is 64 rows of 256 bytes and B 64 k-rows of 256
    // bytes, 16 direct loads of 4 rows each: wave w issues instructions
    // 2w and 2w + 1 of each.
    auto issue = [&](int slot) {
        const int k0 = min(slot, steps - 1) * kQK;
        const float* st = ldsF + (slot % kQStages) * kQStage;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ins = wave * 2 + j;
            const int row = ins * 4 + (lane >> 4);
            const int c = (lane & 15) ^ (row & 15);
            dmaLoad16(reinterpret_cast<const _Float16*>(A + (row0 + row) * lda + k0 + c * 4),
                      reinterpret_cast<const _Float16*>(st + ins * 256));
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ins = wave * 2 + j;
            const int krow = ins * 4 + (lane >> 4);
            dmaLoad16(reinterpret_cast<const _Float16*>(B + static_cast<int64_t>(k0 + krow) * ldb + col0 +
                                                        (lane & 15) * 4),
                      reinterpret_cast<const _Float16*>(st + kQA + ins * 256));
        }
    };
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < kQStages - 1; ++s) issue(s);
    const int l32 = lane & 31, hl = lane >> 5;
    const int m = wm * 32 + l32;
    // A: row m, chunks 8 hl + 4 h .. + 3 (k 32 hl + 16 h .. + 15) at their
    // slots.
    uint32_t offA[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = 4 * h + i;
        offA[i] = 4u * static_cast<uint32_t>(m * kQK + (((8 * hl + q) ^ (m & 15)) * 4));
    }
    // B: k-row 32 hl + 16 h + t, column wn * 32 + l32.
    const uint32_t offB = 4u * static_cast<uint32_t>(kQA + (32 * hl + 16 * h) * kFN + wn * 32 + l32);
    const uint32_t ldsBase = ldsOffset(ldsF);
    // Stage 0 landed (stages 1 and 2, 4 direct loads each per wave, may be
    // in flight).
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    for (int s = 0; s < steps; ++s) {
        const uint32_t cb = ldsBase + 4u * static_cast<uint32_t>((s % kQStages) * kQStage);
        f32x4 a[4];
        float b[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(cb + offA[i]);
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            b[t] = *reinterpret_cast<const __attribute__((address_space(3))) float*>(cb + offB + 4u * kFN * t);
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t >> 2][t & 3], b[t], acc, 0, 0, 0);
        // Stage s + 1 landed (one later stage may be in flight); after the
        // barrier every wave is past step s, so slot (s + 3) % 4, which held
        // step s - 1, can be refilled.
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        asm volatile("s_barrier" ::: "memory");
        issue(s + kQStages - 1);
    }
    // No direct load may still be writing LDS when the halves meet there.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    float* red = ldsF + quad * (64 * 16);
    if (h == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[r * 64 + lane] = acc[r];
    }
    __syncthreads();
    if (h == 1) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] += red[r * 64 + lane];
    if (ACC && skipZeroA && waveNonFinite(acc)) {
        exactWaveBlock<float, float>(A, B, C, lda, ldb, ldc, K, row0 + wm * 32, col0 + wn * 32, 32, 32, ACC);
        return;
    }
    const int64_t cBase = col0 + wn * 32 + l32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t row = row0 + wm * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
        float* dst = C + row * ldc + cBase;
        *dst = ACC ? *dst + acc[r] : acc[r];
    }
}

// ------------------------------------------------------------- general ---
template <typename T>
__device__ __forceinline__ T ldAny(const void* p, int dt, int64_t i) {
    if (dt == MLKD_F32) return static_cast<T>(static_cast<const float*>(p)[i]);
    if (dt == MLKD_F16) return static_cast<T>(static_cast<float>(static_cast<const _Float16*>(p)[i]));
    return static_cast<T>(static_cast<const double*>(p)[i]);
}

template <typename T>
__device__ __forceinline__ void stAny(void* p, int dt, int64_t i, T v) {
    if (dt == MLKD_F32) {
        static_cast<float*>(p)[i] = static_cast<float>(v);
    } else if (dt == MLKD_F16) {
        if constexpr (sizeof(T) == sizeof(double)) static_cast<_Float16*>(p)[i] = mlk::toHalf(v);
        else static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
    } else {
        static_cast<double*>(p)[i] = static_cast<double>(v);
    }
}

/// One 64x64 output tile by 256 threads, 4x4 per thread, K slabs of 16
/// through LDS; k ascending per output element, starting from C's old value
/// in the accumulate form (the reference's order, kernel_buffers.cpp:
/// 406-432). With skip_zero_a the products of A[i,p] == 0 are left out, as
/// there (:422).
template <typename T>
__device__ __forceinline__ void generalTile(const mlkd_gemm& p, int64_t row0, int64_t col0, T (&As)[16][65],
                                            T (&Bs)[16][65]) {
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    T acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = row0 + ty * 4 + i, c = col0 + tx * 4 + j;
            acc[i][j] = (p.accumulate && r < p.m && c < p.n) ? ldAny<T>(p.c, p.c_dtype, r * p.ldc + c) : T(0);
        }
    }
    const bool skip = p.skip_zero_a != 0;
    for (int64_t k0 = 0; k0 < p.k; k0 += 16) {
        for (int e = threadIdx.x; e < 16 * 64; e += 256) {
            const int kk = e / 64, mm = e % 64;
            const int64_t r = row0 + mm, kA = k0 + kk;
            As[kk][mm] = (r < p.m && kA < p.k) ? ldAny<T>(p.a, p.a_dtype, r * p.lda + kA) : T(0);
            const int64_t c = col0 + mm;
            Bs[kk][mm] = (c < p.n && kA < p.k) ? ldAny<T>(p.b, p.b_dtype, kA * p.ldb + c) : T(0);
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            T a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (skip && a[i] == T(0)) continue;
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = row0 + ty * 4 + i, c = col0 + tx * 4 + j;
            if (r < p.m && c < p.n) stAny<T>(p.c, p.c_dtype, r * p.ldc + c, acc[i][j]);
        }
    }
}

/// Any shape and dtype mix: one 64x64 tile per workgroup.
template <typename T>
__global__ __launch_bounds__(256) void gemmGeneral(mlkd_gemm p) {
    __shared__ T As[16][65];
    __shared__ T Bs[16][65];
    const int64_t tilesN = (p.n + 63) / 64;
    generalTile<T>(p, (blockIdx.x / tilesN) * 64, (blockIdx.x % tilesN) * 64, As, Bs);
}

/// Zeroes n 32-bit words.
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Process default of the f16 GEMM launch form (a launch's own `variant`
// field overrides it): 0: 8 waves of 128x64; 1: 4 waves of 128x128; 2: 4
// waves with A direct to LDS; 3: 4 waves, explicitly pipelined; 5/6:
// 128x256 tiles, two workgroups per CU, loads two / one step ahead;
// 7: 4 waves, both operands direct to a 4-deep LDS ring, B read transposed;
// 8: variant 7's data path with 8 waves of 16x16x32 MFMA tiles (measured
// fastest on gfx950).
int gGemmF16Variant = 8;

/// Raises the dynamic-LDS limit of every form that needs more than the
/// default, once per process (a function-local static: its initialization
/// is thread-safe); returns 0 or MLKD_RT_LAUNCH.
int raiseLdsLimits() {
    static const int rc = [] {
        struct Need {
            const void* fn;
            size_t bytes;
        };
        const size_t ldsBytes = 4 * kTileHalves * sizeof(_Float16);
        const size_t ldsDirect = (2 * kTileA + 2 * kTileHalves) * sizeof(_Float16);
        const Need needs[] = {
            {reinterpret_cast<const void*>(gemmF16Mfma<true>), ldsBytes},
            {reinterpret_cast<const void*>(gemmF16Mfma<false>), ldsBytes},
            {reinterpret_cast<const void*>(gemmF16Mfma4w<true>), ldsBytes},
            {reinterpret_cast<const void*>(gemmF16Mfma4w<false>), ldsBytes},
            {reinterpret_cast<const void*>(gemmF16Mfma4wDirect<true>), ldsDirect},
            {reinterpret_cast<const void*>(gemmF16Mfma4wDirect<false>), ldsDirect},
            {reinterpret_cast<const void*>(gemmF16Mfma4wPipe<true>), ldsDirect},
            {reinterpret_cast<const void*>(gemmF16Mfma4wPipe<false>), ldsDirect},
            {reinterpret_cast<const void*>(gemmF16Dma<true>), kLdsDma},
            {reinterpret_cast<const void*>(gemmF16Dma<false>), kLdsDma},
            {reinterpret_cast<const void*>(gemmF16Dma8<true>), kLdsDma},
            {reinterpret_cast<const void*>(gemmF16Dma8<false>), kLdsDma},
            {reinterpret_cast<const void*>(gemmF16Dma8s<true>), kLdsDma},
            {reinterpret_cast<const void*>(gemmF16Dma8s<false>), kLdsDma},
            {reinterpret_cast<const void*>(gemmF32Dma<true>), kLdsF32Dma},
            {reinterpret_cast<const void*>(gemmF32Dma<false>), kLdsF32Dma},
        };
        for (const Need& n : needs) {
            if (hipFuncSetAttribute(n.fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(n.bytes)) !=
                hipSuccess) {
                return static_cast<int>(MLKD_RT_LAUNCH);
            }
        }
        return 0;
    }();
    return rc;
}

/// The MFMA form a launch takes: the f16 form (0-3, 5-8) or 100 + the f32
/// form (0, 1); -1 when the shape, dtypes or alignment fit none of them.
int mfmaForm(const mlkd_gemm* p) {
    const bool fits32 = p->m < (1LL << 31) && p->n < (1LL << 31) && p->k < (1LL << 31);
    if (p->k <= 0 || !fits32) return -1;
    if (p->a_dtype == MLKD_F16 && p->b_dtype == MLKD_F16 && p->c_dtype == MLKD_F32 && p->m % kBM == 0 &&
        p->n % kBN == 0 && p->k % kBK == 0 && p->lda % 8 == 0 && p->ldb % 8 == 0 && aligned16(p->a) &&
        aligned16(p->b)) {
        const int v = p->variant >= 0 ? p->variant : gGemmF16Variant;
        if (v == 8) return (p->ldc % 4) == 0 && aligned16(p->c) ? 8 : 7;
        return v == 7 || v == 5 || v == 6 || v == 3 || v == 2 || v == 1 ? v : 0;
    }
    if (p->a_dtype == MLKD_F32 && p->b_dtype == MLKD_F32 && p->c_dtype == MLKD_F32 && p->m % kFM == 0 &&
        p->n % kFN == 0 && p->k % kFK == 0 && p->lda % 4 == 0 && p->ldb % 4 == 0 && aligned16(p->a) &&
        aligned16(p->b)) {
        const int fv = p->variant >= 0 ? p->variant : 0;
        return fv != 1 && p->k % kQK == 0 ? 100 : 101;
    }
    return -1;
}

/// Form 8 takes gemmF16Dma8s when its lane offsets fit 32 bits and
/// gemmF16Dma8 otherwise; the two give identical results.
bool scalarAddressed8(const mlkd_gemm* p) {
    return p->lda < (int64_t{1} << 23) && p->ldb < (int64_t{1} << 25);
}

int launchMfma(const mlkd_gemm* p, int form, hipStream_t st) {
    const int skip = p->skip_zero_a != 0 ? 1 : 0;
    if (raiseLdsLimits() != 0) return MLKD_RT_LAUNCH;
    const _Float16* a16 = static_cast<const _Float16*>(p->a);
    const _Float16* b16 = static_cast<const _Float16*>(p->b);
    float* c = static_cast<float*>(p->c);
    const int m = static_cast<int>(p->m), n = static_cast<int>(p->n), k = static_cast<int>(p->k);
    const bool acc = p->accumulate != 0;
    const int tiles = static_cast<int>((p->m / kBM) * (p->n / kBN));
    const size_t ldsBytes = 4 * kTileHalves * sizeof(_Float16);
    const size_t ldsDirect = (2 * kTileA + 2 * kTileHalves) * sizeof(_Float16);
    switch (form) {
        case 8:
            if (scalarAddressed8(p)) {
                hipLaunchKernelGGL((acc ? gemmF16Dma8s<true> : gemmF16Dma8s<false>), dim3(tiles), dim3(512), kLdsDma,
                                   st, a16, b16, c, m, n, k, p->lda, p->ldb, p->ldc, skip);
            } else {
                hipLaunchKernelGGL((acc ? gemmF16Dma8<true> : gemmF16Dma8<false>), dim3(tiles), dim3(512), kLdsDma,
                                   st, a16, b16, c, m, n, k, p->lda, p->ldb, p->ldc, skip);
            }
            break;
        case 7:
            hipLaunchKernelGGL((acc ? gemmF16Dma<true> : gemmF16Dma<false>), dim3(tiles), dim3(256), kLdsDma, st,
                               a16, b16, c, m, n, k, p->lda, p->ldb, p->ldc, skip);
            break;
        case 5:
        case 6: {
            const int tiles2 = static_cast<int>((p->m / kBM2) * (p->n / kBN2));
            auto kern = form == 5 ? (acc ? gemmF16Mfma2cu<true, true> : gemmF16Mfma2cu<false, true>)
                                  : (acc ? gemmF16Mfma2cu<true, false> : gemmF16Mfma2cu<false, false>);
            hipLaunchKernelGGL(kern, dim3(tiles2), dim3(256), kLdsGemm2, st, a16, b16, c, m, n, k, p->lda, p->ldb,
                               p->ldc, skip);
            break;
        }
        case 3:
            hipLaunchKernelGGL((acc ? gemmF16Mfma4wPipe<true> : gemmF16Mfma4wPipe<false>), dim3(tiles), dim3(256),
                               ldsDirect, st, a16, b16, c, m, n, k, p->lda, p->ldb, p->ldc, skip);
            break;
        case 2:
            hipLaunchKernelGGL((acc ? gemmF16Mfma4wDirect<true> : gemmF16Mfma4wDirect<false>), dim3(tiles),
                               dim3(256), ldsDirect, st, a16, b16, c, m, n, k, p->lda, p->ldb, p->ldc, p->accumulate,
                               skip);
            break;
        case 1:
            hipLaunchKernelGGL((acc ? gemmF16Mfma4w<true> : gemmF16Mfma4w<false>), dim3(tiles), dim3(256), ldsBytes,
                               st, a16, b16, c, m, n, k, p->lda, p->ldb, p->ldc, p->accumulate, skip);
            break;
        case 0:
            hipLaunchKernelGGL((acc ? gemmF16Mfma<true> : gemmF16Mfma<false>), dim3(tiles), dim3(512), ldsBytes, st,
                               a16, b16, c, m, n, k, p->lda, p->ldb, p->ldc, p->accumulate, skip);
            break;
        case 100:
        case 101: {
            const int ftiles = static_cast<int>((p->m / kFM) * (p->n / kFN));
            const float* a32 = static_cast<const float*>(p->a);
            const float* b32 = static_cast<const float*>(p->b);
            if (form == 100) {
                hipLaunchKernelGGL((acc ? gemmF32Dma<true> : gemmF32Dma<false>), dim3(ftiles), dim3(512), kLdsF32Dma,
                                   st, a32, b32, c, n, k, p->lda, p->ldb, p->ldc, skip);
            } else {
                hipLaunchKernelGGL((acc ? gemmF32Mfma<true> : gemmF32Mfma<false>), dim3(ftiles), dim3(256), 0, st,
                                   a32, b32, c, m, n, k, p->lda, p->ldb, p->ldc, p->accumulate, skip);
            }
            break;
        }
        default:
            return MLKD_RT_LAUNCH;
    }
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

/// dst[r, c] = src[r * lds + c] for r < rows, c < cols, and 0 on the rest
/// of the drows x dcols block (row-major, stride dcols). Element bits are
/// copied as they are (T is a 16- or 32-bit integer type).
template <typename T>
__global__ __launch_bounds__(256) void padBlock(const T* __restrict__ src, int64_t rows, int64_t cols,
                                                int64_t lds, T* __restrict__ dst, int64_t drows, int64_t dcols) {
    for (int64_t r = blockIdx.y; r < drows; r += gridDim.y) {
        for (int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; c < dcols;
             c += static_cast<int64_t>(gridDim.x) * 256) {
            dst[r * dcols + c] = (r < rows && c < cols) ? src[r * lds + c] : T(0);
        }
    }
}

/// dst[r * ldd + c] = src[r * scols + c] for r < rows, c < cols.
template <typename T>
__global__ __launch_bounds__(256) void unpadBlock(const T* __restrict__ src, int64_t scols, T* __restrict__ dst,
                                                  int64_t rows, int64_t cols, int64_t ldd) {
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        for (int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; c < cols;
             c += static_cast<int64_t>(gridDim.x) * 256) {
            dst[r * ldd + c] = src[r * scols + c];
        }
    }
}

/// The zero-padded shape a GEMM the MFMA forms do not tile runs at: f16
/// operands with an f32 C on 256 x 256 tiles, or all-f32 on 64 x 64 tiles,
/// K rounded up to 64. Padding adds only products 0 * 0 to the sums (and
/// the skip-zero-A test skips them), so each output keeps its value. Below
/// 2^30 flop the copies cost more than the general kernel takes.
struct PadShape {
    int64_t m, n, k;
    size_t es;   // operand element bytes
};

bool padShape(const mlkd_gemm* p, PadShape& ps) {
    const bool f16 = p->a_dtype == MLKD_F16 && p->b_dtype == MLKD_F16 && p->c_dtype == MLKD_F32;
    const bool f32 = p->a_dtype == MLKD_F32 && p->b_dtype == MLKD_F32 && p->c_dtype == MLKD_F32;
    if (!(f16 || f32) || p->m <= 0 || p->n <= 0 || p->k <= 0) return false;
    if (p->skip_zero_a != 0 && p->accumulate == 0) return false;   // that launch takes the general kernel
    if (mfmaForm(p) >= 0) return false;                             // already tiled
    const int64_t tm = f16 ? kBM : kFM, tn = f16 ? kBN : kFN, tk = 64;
    ps.m = (p->m + tm - 1) / tm * tm;
    ps.n = (p->n + tn - 1) / tn * tn;
    ps.k = (p->k + tk - 1) / tk * tk;
    ps.es = f16 ? 2 : 4;
    if (ps.m >= (int64_t{1} << 31) || ps.n >= (int64_t{1} << 31) || ps.k >= (int64_t{1} << 31)) return false;
    // Padded when the product is large (2^30 flop and up) or the padding at
    // most 8 times the work: the general kernel takes 36 us at 100^3 and
    // 150 us at 500^3, the padded MFMA launch tens of us at either. Thin
    // shapes padded further (a few rows against 256-row tiles) stay on the
    // general kernel, whose work is then small.
    const double work = static_cast<double>(p->m) * static_cast<double>(p->n) * static_cast<double>(p->k);
    const double padded = static_cast<double>(ps.m) * static_cast<double>(ps.n) * static_cast<double>(ps.k);
    return 2.0 * work >= static_cast<double>(int64_t{1} << 30) || padded <= 8.0 * work;
}

size_t align256g(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

size_t padBytes(const PadShape& ps) {
    return align256g(static_cast<size_t>(ps.m * ps.k) * ps.es) + align256g(static_cast<size_t>(ps.k * ps.n) * ps.es) +
           align256g(static_cast<size_t>(ps.m * ps.n) * sizeof(float));
}

/// The padded launch's MFMA parameters, with A', B', C' carved from the
/// workspace; false when the workspace is missing or too small.
bool paddedParams(const mlkd_gemm* p, mlkd_gemm& q, PadShape& ps) {
    if (p->work == nullptr || !padShape(p, ps) || p->work_bytes < static_cast<int64_t>(padBytes(ps))) return false;
    unsigned char* w = static_cast<unsigned char*>(p->work);
    q = *p;
    q.a = w;
    q.b = w + align256g(static_cast<size_t>(ps.m * ps.k) * ps.es);
    q.c = static_cast<unsigned char*>(const_cast<void*>(q.b)) + align256g(static_cast<size_t>(ps.k * ps.n) * ps.es);
    q.m = ps.m;
    q.n = ps.n;
    q.k = ps.k;
    q.lda = ps.k;
    q.ldb = ps.n;
    q.ldc = ps.n;
    q.work = nullptr;
    q.work_bytes = 0;
    return mfmaForm(&q) >= 0;
}

/// padBlock in 16-byte pieces, for source rows that start 16-byte aligned
/// (src and lds * sizeof(T) multiples of 16; dcols a multiple of 16 /
/// sizeof(T)). A piece that straddles `cols` is copied element by element.
template <typename T>
__global__ __launch_bounds__(256) void padBlock16(const T* __restrict__ src, int64_t rows, int64_t cols,
                                                  int64_t lds, T* __restrict__ dst, int64_t drows, int64_t dcols) {
    constexpr int V = 16 / sizeof(T);
    const int64_t pieces = dcols / V;
    for (int64_t r = blockIdx.y; r < drows; r += gridDim.y) {
        for (int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; j < pieces;
             j += static_cast<int64_t>(gridDim.x) * 256) {
            const int64_t c0 = j * V;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (r < rows && c0 + V <= cols) {
                v = *reinterpret_cast<const u32x4*>(src + r * lds + c0);
            } else if (r < rows && c0 < cols) {
                T e[V];
#pragma unroll
                for (int i = 0; i < V; ++i) e[i] = c0 + i < cols ? src[r * lds + c0 + i] : T(0);
                v = __builtin_bit_cast(u32x4, e);
            }
            *reinterpret_cast<u32x4*>(dst + r * dcols + c0) = v;
        }
    }
}

/// unpadBlock in 16-byte pieces (dst and ldd * 4 multiples of 16 bytes); a
/// piece that straddles `cols` is copied element by element.
__global__ __launch_bounds__(256) void unpadBlock16(const uint32_t* __restrict__ src, int64_t scols,
                                                    uint32_t* __restrict__ dst, int64_t rows, int64_t cols,
                                                    int64_t ldd) {
    const int64_t pieces = (cols + 3) / 4;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        for (int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; j < pieces;
             j += static_cast<int64_t>(gridDim.x) * 256) {
            const int64_t c0 = j * 4;
            if (c0 + 4 <= cols) {
                *reinterpret_cast<u32x4*>(dst + r * ldd + c0) = *reinterpret_cast<const u32x4*>(src + r * scols + c0);
            } else {
                for (int64_t c = c0; c < cols; ++c) dst[r * ldd + c] = src[r * scols + c];
            }
        }
    }
}

template <typename T>
void launchPad(const void* src, int64_t rows, int64_t cols, int64_t lds, void* dst, int64_t drows, int64_t dcols,
               hipStream_t st) {
    constexpr int V = 16 / sizeof(T);
    const unsigned gy = static_cast<unsigned>(std::min<int64_t>(drows, 4096));
    if ((reinterpret_cast<uintptr_t>(src) & 15) == 0 && (lds * static_cast<int64_t>(sizeof(T))) % 16 == 0 &&
        dcols % V == 0) {
        const unsigned gx = static_cast<unsigned>(std::min<int64_t>((dcols / V + 255) / 256, 64));
        hipLaunchKernelGGL(padBlock16<T>, dim3(gx, gy), dim3(256), 0, st, static_cast<const T*>(src), rows, cols, lds,
                           static_cast<T*>(dst), drows, dcols);
        return;
    }
    const unsigned gx = static_cast<unsigned>(std::min<int64_t>((dcols + 255) / 256, 64));
    hipLaunchKernelGGL(padBlock<T>, dim3(gx, gy), dim3(256), 0, st, static_cast<const T*>(src), rows, cols, lds,
                       static_cast<T*>(dst), drows, dcols);
}

int launchPadded(const mlkd_gemm* p, const mlkd_gemm& q, const PadShape& ps, hipStream_t st) {
    if (ps.es == 2) {
        launchPad<uint16_t>(p->a, p->m, p->k, p->lda, const_cast<void*>(q.a), ps.m, ps.k, st);
        launchPad<uint16_t>(p->b, p->k, p->n, p->ldb, const_cast<void*>(q.b), ps.k, ps.n, st);
    } else {
        launchPad<uint32_t>(p->a, p->m, p->k, p->lda, const_cast<void*>(q.a), ps.m, ps.k, st);
        launchPad<uint32_t>(p->b, p->k, p->n, p->ldb, const_cast<void*>(q.b), ps.k, ps.n, st);
    }
    // C += A*B reads C: its padded copy starts from C (and zeros).
    if (p->accumulate != 0) launchPad<uint32_t>(p->c, p->m, p->n, p->ldc, q.c, ps.m, ps.n, st);
    if (hipGetLastError() != hipSuccess) return MLKD_RT_LAUNCH;
    if (const int rc = launchMfma(&q, mfmaForm(&q), st); rc != 0) return rc;
    const unsigned gy = static_cast<unsigned>(std::min<int64_t>(p->m, 4096));
    if ((reinterpret_cast<uintptr_t>(p->c) & 15) == 0 && p->ldc % 4 == 0) {
        const unsigned gx = static_cast<unsigned>(std::min<int64_t>(((p->n + 3) / 4 + 255) / 256, 64));
        hipLaunchKernelGGL(unpadBlock16, dim3(gx, gy), dim3(256), 0, st, static_cast<const uint32_t*>(q.c), ps.n,
                           static_cast<uint32_t*>(p->c), p->m, p->n, p->ldc);
    } else {
        const unsigned gx = static_cast<unsigned>(std::min<int64_t>((p->n + 255) / 256, 64));
        hipLaunchKernelGGL(unpadBlock<uint32_t>, dim3(gx, gy), dim3(256), 0, st, static_cast<const uint32_t*>(q.c),
                           ps.n, static_cast<uint32_t*>(p->c), p->m, p->n, p->ldc);
    }
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

}  // namespace

extern "C" void mlkd_gemm_set_variant(int variant) { gGemmF16Variant = variant; }

extern "C" int64_t mlkd_gemm_pad_bytes(const mlkd_gemm* p) {
    PadShape ps;
    return p != nullptr && padShape(p, ps) ? static_cast<int64_t>(padBytes(ps)) : 0;
}

extern "C" const char* mlkd_gemm_kernel_name(const mlkd_gemm* p) {
    {
        // A padded launch is named by the MFMA form it runs.
        mlkd_gemm q;
        PadShape ps;
        if (paddedParams(p, q, ps)) return mlkd_gemm_kernel_name(&q);
    }
    const bool acc = p->accumulate != 0;
    switch (p->skip_zero_a != 0 && !acc ? -1 : mfmaForm(p)) {
        case 8:
            if (scalarAddressed8(p)) return acc ? "gemmF16Dma8s<true>" : "gemmF16Dma8s<false>";
            return acc ? "gemmF16Dma8<true>" : "gemmF16Dma8<false>";
        case 7: return acc ? "gemmF16Dma<true>" : "gemmF16Dma<false>";
        case 6: return acc ? "gemmF16Mfma2cu<true, false>" : "gemmF16Mfma2cu<false, false>";
        case 5: return acc ? "gemmF16Mfma2cu<true, true>" : "gemmF16Mfma2cu<false, true>";
        case 3: return acc ? "gemmF16Mfma4wPipe<true>" : "gemmF16Mfma4wPipe<false>";
        case 2: return acc ? "gemmF16Mfma4wDirect<true>" : "gemmF16Mfma4wDirect<false>";
        case 1: return acc ? "gemmF16Mfma4w<true>" : "gemmF16Mfma4w<false>";
        case 0: return acc ? "gemmF16Mfma<true>" : "gemmF16Mfma<false>";
        case 100: return acc ? "gemmF32Dma<true>" : "gemmF32Dma<false>";
        case 101: return acc ? "gemmF32Mfma<true>" : "gemmF32Mfma<false>";
        default: break;
    }
    const bool wide = p->a_dtype == MLKD_F64 || p->b_dtype == MLKD_F64 || p->c_dtype == MLKD_F64;
    return wide ? "gemmGeneral<double>" : "gemmGeneral<float>";
}

extern "C" int mlkd_launch_gemm(const mlkd_gemm* p, void* stream) {
    if (p == nullptr || p->m < 0 || p->n < 0 || p->k < 0) return MLKD_RT_LAUNCH;
    if (p->m == 0 || p->n == 0) return 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // The MFMA forms take the skip-zero-A Call form themselves: a wave whose
    // accumulators met an infinity or a NaN recomputes its block exactly. One
    // launch, no scratch, no host read-back.
    // Only the accumulating (Call) form skips; a non-accumulating launch that
    // asks for the skip takes the general kernel.
    if (const int form = mfmaForm(p); form >= 0 && (p->skip_zero_a == 0 || p->accumulate != 0)) {
        return launchMfma(p, form, st);
    }
    {
        mlkd_gemm q;
        PadShape ps;
        if (paddedParams(p, q, ps)) {
            if (raiseLdsLimits() != 0) return MLKD_RT_LAUNCH;
            return launchPadded(p, q, ps, st);
        }
    }
    const int64_t tiles = ((p->m + 63) / 64) * ((p->n + 63) / 64);
    if (tiles > 0x7FFFFFFF) return MLKD_RT_LAUNCH;
    const bool wide = p->a_dtype == MLKD_F64 || p->b_dtype == MLKD_F64 || p->c_dtype == MLKD_F64;
    if (wide) {
        hipLaunchKernelGGL(gemmGeneral<double>, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, st, *p);
    } else {
        hipLaunchKernelGGL(gemmGeneral<float>, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, st, *p);
    }
    return hipGetLastError() == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}
