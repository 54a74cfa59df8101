// The thin C ABI between the C++ host code and the HIP side: runtime
// wrappers (runtime.hip) and one launcher per kernel class. Host code includes
// only this header; it never includes HIP headers.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../device_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/// Status codes of the artifact ABI (docs/kernel_abi.md:25-40).
enum {
    MLKD_RT_OK = 0,
    MLKD_RT_NEG_FLAT = 1,
    MLKD_RT_ALLOC = 2,
    MLKD_RT_LAUNCH = 3,
    MLKD_RT_NO_DEVICE = 4,
};

int mlkd_rt_device_count(void);
int mlkd_rt_device_arch(int dev, char* buf, size_t cap);
int mlkd_rt_device_info(int dev, int* cu_count, int64_t* max_grid_x, int* max_block,
                        int64_t* global_mem);
int mlkd_rt_malloc(void** p, size_t bytes);
int mlkd_rt_free(void* p);
/// Page-locked host memory (hipHostMalloc): copies between it and the device
/// run at DMA rate. Released by mlkd_rt_host_free.
int mlkd_rt_host_alloc(void** p, size_t bytes);
int mlkd_rt_host_free(void* p);
int mlkd_rt_h2d(void* dst, const void* src, size_t bytes, void* stream);
int mlkd_rt_d2h(void* dst, const void* src, size_t bytes, void* stream);
int mlkd_rt_d2d(void* dst, const void* src, size_t bytes, void* stream);
int mlkd_rt_fill32(void* p, uint32_t value, size_t bytes, void* stream);
/// The allocation-free entry's device scratch on the current device: its
/// address (hipGetSymbolAddress of the file-scope array, taken once per
/// device) and size. Allocates nothing.
int mlkd_rt_noalloc_scratch(void** ptr, size_t* bytes);
int mlkd_rt_sync(void* stream);
int mlkd_rt_device_sync(void);
int mlkd_rt_stream_create(void** s);
int mlkd_rt_stream_destroy(void* s);
int mlkd_rt_event_create(void** e);
int mlkd_rt_event_destroy(void* e);
int mlkd_rt_event_record(void* e, void* stream);
/* Waits on the host until the work before the event's record has finished. */
int mlkd_rt_event_sync(void* e);
int mlkd_rt_event_elapsed_ms(void* start, void* stop, float* ms);
const char* mlkd_rt_last_error(void);

/// hipRTC instances of kernel templates (jit.hip).
int mlkd_jit_version(int* major, int* minor);
/// The hipRTC option list every instance is compiled with, space-separated
/// into `buf`; returns the option count.
int mlkd_jit_options(const char* arch, char* buf, size_t cap);
int mlkd_jit_build(const char* src, size_t len, const char* name, const char* arch,
                   const char* cache_dir, void** fn_out, uint64_t* fingerprint_out, char* log,
                   size_t cap);
long long mlkd_jit_compile_only(const char* src, size_t len, const char* arch, char* log,
                                size_t cap);
int mlkd_jit_launch_elementwise(void* fn, unsigned grid, const void* const* in, void* out,
                                const mlkd_scalars* scalars, long long dyn_extent, void* stream);

/// Kernel argument block of a generic loop-nest instance (the generated
/// kernel declares the same layout): buffer slots, their element counts, the
/// status word of run-time bounds checks, the run's element count.
typedef struct {
    void* p[16];
    long long n[16];
    int* status;
    long long elements;
} mlkd_nest_args;

/// Launches a loop-nest instance: (mlkd_nest_args, scalars, long long total),
/// `block` threads per workgroup.
int mlkd_jit_launch_nest(void* fn, unsigned grid, unsigned block, const mlkd_nest_args* args,
                         const mlkd_scalars* scalars, long long total, void* stream);
int mlkd_launch_rowsum(const mlkd_softmax* p, void* stream);

/// Kernel launchers (device/*.hip). Each validates nothing beyond launch
/// shape: the host planner has already proved every address in bounds.
int mlkd_launch_softmax(const mlkd_softmax* p, void* stream);
/// Variant-space hook for the softmax launch (0: row per wave with v_exp_f32,
/// 1: pipelined rows over `waves` waves, 2: row per wave with expf, 3/4: 0/2
/// with plain stores; waves <= 0 keeps the default grid).
void mlkd_softmax_set_variant(int variant, int64_t waves);
int mlkd_launch_gemm(const mlkd_gemm* p, void* stream);
/// Bytes of workspace that let mlkd_launch_gemm run `p` on an MFMA form
/// through zero-padded copies of A, B and C; 0 when the shape needs none
/// (already tiled, another dtype combination, or too small to pay for the
/// copies).
int64_t mlkd_gemm_pad_bytes(const mlkd_gemm* p);
/// The symbol of the kernel mlkd_launch_gemm runs for `p` (the MFMA form, or
/// the general kernel), as profilers print it without the parameters. A
/// skip-zero-A launch is the same single kernel.
const char* mlkd_gemm_kernel_name(const mlkd_gemm* p);
/// Likewise for the softmax launch (valid until this thread's next call).
const char* mlkd_softmax_kernel_name(const mlkd_softmax* p);
/// Likewise for score-softmax: its kernels joined by '+' (valid until this
/// thread's next call).
const char* mlkd_score_kernel_names(const mlkd_score_softmax* p);
/// Workspace bytes that let mlkd_launch_score_softmax run a sequence length
/// off the two-pass form's blocks on zero-padded copies; 0 when none applies.
int64_t mlkd_score_pad_bytes(const mlkd_score_softmax* p);
/// Process default of the f16 GEMM launch form (8: direct-to-LDS ring with 8
/// waves of 16x16x32 tiles, the default; 7: the same ring with 4 waves of
/// 32x32x16; 0: 8 waves x 128x64; 1: 4 waves x 128x128; 2: A direct to LDS;
/// 3: pipelined step; 5/6: 128x256 tiles, two workgroups per CU).
void mlkd_gemm_set_variant(int variant);
int mlkd_launch_score_softmax(const mlkd_score_softmax* p, void* stream);
/// Scratch bytes the two-pass score-softmax form needs for `p`'s shape (0 when
/// that form does not apply).
int64_t mlkd_score_scratch_bytes(const mlkd_score_softmax* p);
/// Variant-space hook for score-softmax (0: best form for the shape, 1: scores
/// then softmax, 2: fused single pass, 3: two-pass 256 x 256 blocks, 8:
/// two-pass query-stationary).
void mlkd_score_set_variant(int variant);

/// Measured HBM bandwidth (streaming copy of 256 MiB) and f16 MFMA
/// throughput (register-only MFMAs, one wave per SIMD) of the current
/// device, timed on `stream` (probe.hip).
int mlkd_probe_environment(double* bytes_per_sec, double* f16_flops_per_sec, void* stream);
/// Settled f16 MFMA rate of a register-only loop (probe.hip): shape 0 =
/// 16x16x32, 1 = 32x32x16; random (1) or all-ones (0) operands; 1 or 2 waves
/// per SIMD. Measurement only: calibrates the MFMA-busy counters.
int mlkd_probe_mfma_rate(int shape, int random, int waves_per_simd, double settle_ms, int reps,
                         double* flops_per_sec, void* stream);

#ifdef __cplusplus
}
#endif
