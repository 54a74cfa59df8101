/*
 * mlk_hip.h — C ABI of the MI355X (gfx950) execution backend for MLK+
 * KernelModules (libmlk_hip.so). Plain pointers and sizes only.
 *
 * The backend replaces the reference's GPU artifact path:
 *   buildGpuKernelArtifact[InDir] / LoadedKernel / cudaToolchainAvailable
 *     backends/cpu/include/mlk/backend/backend_driver.h:91-228
 *   the generated artifact's mlk_kernel entry (multi-dim and legacy 1-D)
 *     docs/kernel_abi.md:25-40, backend_driver.h:15-46,
 *     backends/cpu/src/cuda_emitter.cpp:1130-1375, :1762-1867
 *   cudaArtifactBitExactPolicy
 *     backends/cpu/include/mlk/backend/cuda_emitter.h:106-137
 * A module crosses the boundary as the "mlk-kernel" JSON document that
 * KernelModule::toJson writes (compiler/src/support/kernel_ir.cpp:97-254),
 * with "math" also written on Call nodes.
 *
 * Status codes (artifact ABI, docs/kernel_abi.md:25-40): 0 ok, 1 negative
 * store address, 2 runtime allocation/copy, 3 launch or synchronization,
 * 4 no usable device. Extensions: 6 binding mismatch (wrong count, dtype or
 * size), 7 module refused at build (see mlkhip_last_error).
 */
#ifndef MLK_HIP_H
#define MLK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MLKHIP_OK = 0,
    MLKHIP_NEG_STORE = 1,
    MLKHIP_RUNTIME = 2,
    MLKHIP_LAUNCH = 3,
    MLKHIP_NO_DEVICE = 4,
    MLKHIP_BAD_BINDING = 6,
    MLKHIP_REFUSED = 7
};

/* Device element types (KernelBuffer::dtype subset). */
enum { MLKHIP_F32 = 0, MLKHIP_F16 = 1, MLKHIP_F64 = 2 };

typedef struct mlkhip_artifact mlkhip_artifact;

/* One device-resident buffer of the typed entry point. */
typedef struct mlkhip_binding {
    void* ptr;          /* device address; NULL for a temp lets the artifact own it */
    int64_t elements;   /* capacity in elements */
    int32_t dtype;      /* MLKHIP_F32 / MLKHIP_F16 / MLKHIP_F64, must equal the module's */
    int32_t pad;
} mlkhip_binding;

/* ---- driver (replaces backend_driver.h:91-228) ------------------------ */

/* Message of the last failing call on this thread. */
const char* mlkhip_last_error(void);

/* Replaces cudaToolchainAvailable (backend_driver.h:98-104): 1 when a HIP
 * device is visible and its architecture starts with `arch`. */
int mlkhip_device_available(const char* arch);

/* Replaces validArch (backend_driver.cpp:693-699) for AMD targets: 1 when
 * `arch` is gfx followed by 3 or 4 hex digits (gfx950, gfx90a, gfx1100). */
int mlkhip_valid_arch(const char* arch);

/* Replaces buildGpuKernelArtifact[InDir] (backend_driver.h:218-228): plans
 * the module onto the gfx950 kernels, instantiates and compiles the
 * template kernels it needs (hipRTC, cached in `cache_dir` when given) and
 * loads them. `arch` is declared, never defaulted. */
int mlkhip_build(const char* module_json, size_t len, const char* arch, const char* cache_dir,
                 mlkhip_artifact** out);

/* Plans without compiling or loading (no device needed). Writes the class
 * and policy names; returns 0 or MLKHIP_REFUSED. */
int mlkhip_plan(const char* module_json, size_t len, char* class_name, size_t class_cap,
                char* policy, size_t policy_cap, int* n_steps);

/* The hipRTC options every instance is compiled with for `arch` (target,
 * -O3, -std=c++17, -ffp-contract=off, packed FP32 instructions disabled),
 * space-separated into `buf`; returns the option count. No device needed. */
int mlkhip_jit_options(const char* arch, char* buf, size_t cap);

/* Instantiates the hipRTC source of step `step` (elementwise and generic
 * loop-nest steps) and compiles it for `arch` without loading; returns the
 * code-object size, 0 for steps that use precompiled kernels, or -1.
 * `source` may be NULL. */
long long mlkhip_compile_check(const char* module_json, size_t len, int step, const char* arch,
                               char* source, size_t source_cap);

/* Replaces buildGpuKernelArtifactInDir (backend_driver.h:218-228) in its
 * file-backed form: writes <dir>/mlk_kernel.cpp, a per-module artifact that
 * exports `mlk_kernel` exactly as LoadedKernel::run binds it (dlsym at
 * backend_driver.cpp:427, typed call at :932-1042; docs/kernel_abi.md:25-40):
 *   multi-dim:  int mlk_kernel(<T0> p0, const int64_t* p0_dims, ...,
 *                              const double* mlk_scalars, int64_t mlk_n_scalars)
 *   legacy 1-D: void mlk_kernel(<T0> p0, ..., int64_t n,
 *                               const double* mlk_scalars, int64_t mlk_n_scalars)
 * (<Ti> = double* for stored, output and temp buffers, const double*
 * otherwise; one entry per bindable buffer in table order; temp slots are
 * ignored) plus `int mlk_kernel_status(void)`, the calling thread's last
 * status (the legacy form's side channel). Each call forwards to
 * mlkhip_kernel / mlkhip_kernel_1d of this library; the first call builds
 * the embedded module for the embedded `arch`. The source is compiled out of
 * process with `compiler` (NULL or "": c++) into <dir>/libmlk_kernel.so,
 * linked against this library; its path goes to `path_out`. The module is
 * planned first, so what mlkhip_build refuses is refused here
 * (MLKHIP_REFUSED, see mlkhip_last_error). No device needed. */
int mlkhip_emit_artifact(const char* module_json, size_t len, const char* arch, const char* compiler,
                         const char* dir, char* path_out, size_t cap);

void mlkhip_release(mlkhip_artifact* a);

/* No counterpart in the reference (its artifact allocates per call): frees
 * the scratch set mlkhip_run_device keeps for `stream` (temps, row
 * statistics), after waiting for that stream. A caller that
 * runs an artifact on many short-lived streams releases each one's set
 * before destroying the stream; the next run on a released stream
 * allocates a new set. Must not overlap a run of `a` on `stream` from
 * another thread. Returns 0, or MLKHIP_LAUNCH when the wait fails. */
int mlkhip_release_stream_scratch(mlkhip_artifact* a, void* stream);

int mlkhip_is_multidim(const mlkhip_artifact* a);
const char* mlkhip_class_name(const mlkhip_artifact* a);

/* Replaces cudaArtifactBitExactPolicy (cuda_emitter.h:106-137): the
 * tolerance policy id the artifact's results are certified under. */
const char* mlkhip_policy(const mlkhip_artifact* a);

/* Number of bindable buffers (input | output | temp, table order) and the
 * module's dtype / element count of bindable `i` (elements = -1 when the
 * buffer is sized by the run's dynamic element count). */
int mlkhip_num_bindables(const mlkhip_artifact* a);
int mlkhip_bindable_info(const mlkhip_artifact* a, int i, int32_t* dtype, int64_t* elements,
                         int* is_input, int* is_output, int* is_temp);

/* ---- artifact ABI (docs/kernel_abi.md:25-40) --------------------------- */

/* Multi-dim form: one (f64 host pointer, dims) pair per bindable buffer in
 * table order (temps: pass NULL; the artifact materializes zeroed device
 * scratch), the scalar table, the dynamic element count. Converts to the
 * module dtypes (RNE) on upload, back to f64 on download; outputs are
 * uploaded too, since += and max stores read them. Synchronous. The copies
 * go through up to 64 MiB of page-locked staging that the artifact keeps
 * until it is released, in two halves so that converting one chunk overlaps
 * copying the previous one; host-buffer calls on one artifact run one at a
 * time. */
int mlkhip_kernel(const mlkhip_artifact* a, double* const* ptrs, const int64_t* const* dims,
                  int n_bindables, const double* scalars, int64_t n_scalars, int64_t elements);

/* Legacy 1-D form (the reference's void mlk_kernel(..., int64_t n, scalars)):
 * bindable pointers in table order, n = element count. Returns a status
 * instead of swallowing it. */
int mlkhip_kernel_1d(const mlkhip_artifact* a, double* const* ptrs, int n_ptrs, int64_t n,
                     const double* scalars, int64_t n_scalars);

/* Device-resident typed entry (the timing path): no copies, no allocation
 * except artifact-owned scratch (temps, the score-softmax row statistics),
 * one set per stream; enqueued on `stream` (a hipStream_t, NULL = default
 * stream), asynchronous: no step reads anything back to the host except a
 * loop nest with run-time bounds checks, which waits for its status word. A
 * Call(MatMul) step decides its skip-zero-A handling on the device
 * (kernel_buffers.cpp:422) in one launch: the skip can change C only where B
 * holds an infinity or a NaN, which makes the MFMA accumulators there
 * non-finite, so a wave that finds one recomputes its block exactly. */
int mlkhip_run_device(const mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds,
                      const double* scalars, int64_t n_scalars, int64_t elements, void* stream);

/* No counterpart in the reference: the allocation-free variant of
 * mlkhip_run_device, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The caller passes inputs and outputs as for mlkhip_run_device;
 * every scratch buffer the run needs (materialized temps, zeroed on every
 * run, and the score-softmax row statistics) is carved out of one
 * file-scope device array of mlkhip_noalloc_scratch_bytes() bytes (32 MiB)
 * that each GPU holds until the process ends. A run that needs more is
 * refused (MLKHIP_REFUSED, see mlkhip_last_error) before anything is
 * launched, as is a step that needs a host read-back (a loop nest with
 * run-time bounds checks). A Call(MatMul) step runs the same single kernel
 * as mlkhip_run_device and needs none of the array. The entry calls no
 * hipMalloc or hipFree. Every call on one GPU shares that GPU's array,
 * which keeps the last call's contents: calls that overlap on one GPU (on
 * different streams, or from different threads) race. Enqueued on `stream`,
 * asynchronous. */
int mlkhip_run_device_noalloc(const mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds,
                              const double* scalars, int64_t n_scalars, int64_t elements, void* stream);

/* Size in bytes of the allocation-free entry's device array (0 without a
 * device). */
size_t mlkhip_noalloc_scratch_bytes(void);

/* Times `reps` back-to-back launches of the device entry after `warmup`
 * untimed ones, with HIP events on `stream`; writes per-launch milliseconds
 * (reps values) into `ms_out`. */
int mlkhip_time_device(const mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds,
                       const double* scalars, int64_t n_scalars, int64_t elements, void* stream,
                       int warmup, int reps, float* ms_out);

/* Times `reps` back-to-back launches with one HIP event pair around the
 * whole span on `stream` (after `warmup` untimed launches) and writes the
 * average milliseconds per launch into `avg_ms`. */
int mlkhip_time_device_span(const mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds,
                            const double* scalars, int64_t n_scalars, int64_t elements, void* stream,
                            int warmup, int reps, float* avg_ms);

/* ---- launch-form search (fastkernel on the gfx950 kernels) ------------ */
/* The reference's fastkernel search (fastkernel/include/mlk/fastkernel/
 * fast_kernel.h:165-355, src/fast_kernel.cpp:797-887) certifies tile and
 * exec-path variants of a kernel and keeps the fastest. Here the declared
 * space is the launch forms of each step's kernel: softmax rows (exp form,
 * store cache policy, pipelining), f16 GEMM tiles and schedules, the f32
 * GEMM's operand staging, score-softmax pass structure, and the generic
 * loop-nest kernel's LDS slabs, workgroup size (256, 512, 64) and collapse
 * depth. */

/* Number of steps (kernel launches) of the artifact's plan. */
int mlkhip_num_steps(const mlkhip_artifact* a);

/* Declared variant space of step `step` (VariantConfig, fast_kernel.h:
 * 170-174): writes up to `cap` form ids into `out` (may be NULL) and
 * returns how many there are (0 = only the default form) or -1. The first
 * id is the kernel's default form. */
int mlkhip_step_variants(const mlkhip_artifact* a, int step, int* out, int cap);

/* The same without a device: plans the module and lists step `step`'s
 * variant space. */
int mlkhip_plan_variants(const char* module_json, size_t len, int step, int* out, int cap);

/* Kernel symbol of step `step`, as profiles name kernels: a hipRTC
 * instance's (an elementwise chain: mlk_elementwise_<12 hex digits of its
 * source hash>; a generic loop nest: mlk_nest), or the precompiled kernel
 * the step's launcher picks for its shape, dtypes and pinned form on
 * 256-byte aligned buffers, with template arguments and without parameters
 * (gemmF16Dma8s<true>, softmaxWaveRowPair<16, true>; a two-kernel launch
 * joins them with '+': scoreStatsQ+scoreStoreQ). The text lives as long as
 * the artifact. */
const char* mlkhip_step_kernel_name(const mlkhip_artifact* a, int step);

/* Form step `step` launches with (-1 = the kernel's default); -2 when the
 * step does not exist. */
int mlkhip_step_variant(const mlkhip_artifact* a, int step);

/* Pins step `step` to form `variant` (-1 = default). Returns 0, or
 * MLKHIP_BAD_BINDING for a step or form outside the declared space. */
int mlkhip_set_step_variant(mlkhip_artifact* a, int step, int variant);

/* Completeness fingerprint of the artifact's cache entry (fast_kernel.cpp:
 * 727-763): module hash, declared target, hipRTC version, policy, device.
 * 16 hex digits. */
const char* mlkhip_fingerprint(const mlkhip_artifact* a);

/* 1 when mlkhip_build applied a cached choice (<cache_dir>/fk-<fingerprint>
 * .json) to the steps; the reference's cacheHits (fast_kernel.h:345-346). */
int mlkhip_variants_from_cache(const mlkhip_artifact* a);

/* Replaces runFastKernelSearch (fast_kernel.h:355-357) for the artifact's
 * own launch forms. On the caller's device buffers (bindings as for
 * mlkhip_run_device): runs every step in its default form as the
 * reference; for each step with more than one form, runs each form with the
 * other steps at default, certifies it when its outputs are within half of
 * the artifact's tolerance policy of the reference's (bit-identical under a
 * bit-exact policy; the identity gate of fast_kernel.cpp:1251-1261), times
 * `reps` single launches after 2 warmups and takes the median (fast_kernel
 * .cpp:697-719); keeps the fastest certified form per step and certifies the
 * chosen combination as a whole (falling back to all defaults if it fails).
 * The buffers the artifact writes are snapshotted before and restored after
 * the search. When `cache_dir` is not NULL or empty the choice is written to
 * <cache_dir>/fk-<fingerprint>.json, which mlkhip_build with the same
 * cache_dir applies. `report` (may be NULL) receives a JSON document of every
 * candidate with its certificate or rejection (FastKernelReport::toJson,
 * fast_kernel.cpp:940-1040). Synchronous; returns a status code. */
int mlkhip_autotune(mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds, const double* scalars,
                    int64_t n_scalars, int64_t elements, int reps, const char* cache_dir, char* report,
                    size_t report_cap);

/* Replaces essentialWorkModel + rooflineLowerBound (fastkernel/src/
 * fast_kernel.cpp:319-384, fast_kernel.h:100-117) with element sizes from
 * the buffers' dtypes: min_bytes counts every non-temp input and output
 * once at 8/4/2 bytes per f64/f32/f16 element (the reference counts 8 for
 * all); min_ops follows the reference's walk (MatMul 2MKN, Softmax 5 per
 * element, ReduceSum 1 per element, 1 per Compute expression and per
 * accumulate store, counted once per path from the node list). The lower
 * bound is max(min_bytes / bytes_per_sec, min_ops / ops_per_sec), 0 when a
 * count is unknown (a dynamic extent without dims). bytes_per_sec <= 0
 * takes MI355X HBM (8e12 B/s); ops_per_sec <= 0 takes the datasheet rate
 * of the plan (2.5e15 with an f16 GEMM or score step, 78.6e12 for f64-only
 * modules, else 157.3e12). No device needed. mlkhip_autotune reports the
 * same quantities with its winner's gap over the bound, and a launch
 * coverage certificate per step (certifyLaunchCoverage, fast_kernel.cpp:
 * 386-497, restated for the GPU decomposition). */
int mlkhip_essential_work(const char* module_json, size_t len, double bytes_per_sec, double ops_per_sec,
                          int64_t* min_bytes, int64_t* min_ops, int* bytes_known, int* ops_known,
                          double* roofline_lower_sec);

/* Replaces measureEnvironment (fast_kernel.cpp:319-335, which probes CPU
 * bandwidth and throughput) for the device: HBM bytes/s of a streaming copy
 * of 256 MiB and the f16 MFMA rate of register-only v_mfma_f32_32x32x16_f16
 * loops, one wave per SIMD. Probed once per process (about 30 ms, 512 MiB
 * of temporary device memory); later calls return the same numbers.
 * mlkhip_autotune reports them with the bound they give. */
int mlkhip_measure_environment(double* bytes_per_sec, double* f16_flops_per_sec);

/* ---- run route (the ExecutionEngine hook of `mlkc run`) ---------------- */
/* `mlkc run` reaches only the CPU executor (tools/mlkc/mlkc.cpp:206-263,
 * runtime/src/execution/execution.cpp:195-256). These two entries are what
 * an ExecutionEngine hook behind a `--backend=hip` flag calls in place of
 * the CPU executor, falling back to Tier 0 on any nonzero code. Each builds
 * the module for `arch` on first use and keeps the artifact in a
 * process-wide cache keyed by target and module text. */

/* Replaces executeKernelOnBuffers (runtime/include/mlk/runtime/execution.h:
 * 113-140, kernel_buffers.cpp:839-1106) with KernelBufferBindings spelled
 * out: dense f64 host buffers, an input buffer id indexing `inputs` and an
 * output buffer id indexing `outputs` after the input count, as the
 * reference resolves them (kernel_buffers.cpp:200-230); temps are the
 * artifact's. Outputs are read and written (+= and max stores). An unbound
 * buffer is MLKHIP_BAD_BINDING (the reference would skip its stores).
 * Synchronous; returns a status code. */
int mlkhip_execute_kernel_on_buffers(const char* module_json, size_t len, const char* arch, double* const* inputs,
                                     int n_inputs, double* const* outputs, int n_outputs, const double* scalars,
                                     int64_t n_scalars, int64_t elements);

/* Replaces executeKernel (execution.cpp:195-256), the scalar ABI: inputs
 * are the ScalarParams in value-id order, each output buffer gets its own
 * f64 slots, element 0 of output buffer i goes to output_scalars[i], one
 * instance. A module with input buffers is MLKHIP_REFUSED, as there. */
int mlkhip_execute_kernel(const char* module_json, size_t len, const char* arch, const double* input_scalars,
                          int n_inputs, double* output_scalars, int n_outputs);

/* Number of artifacts the execute entries hold, and releasing them. */
int mlkhip_execute_cache_size(void);
void mlkhip_execute_cache_clear(void);

/* ---- device memory plumbing for hosts without another HIP runtime ----- */
int mlkhip_malloc(void** p, size_t bytes);
int mlkhip_free(void* p);
int mlkhip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int mlkhip_memcpy_d2h(void* dst, const void* src, size_t bytes);
int mlkhip_fill32(void* p, uint32_t value, size_t bytes);
int mlkhip_synchronize(void);
int mlkhip_stream_create(void** s);
int mlkhip_stream_destroy(void* s);

#ifdef __cplusplus
}
#endif

#endif /* MLK_HIP_H */
