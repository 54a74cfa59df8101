// Class recognition: turns a KernelModule into a plan of launches of the
// hand-written gfx950 kernels, with every address proved in bounds on the
// host before anything runs on the device.
#pragma once

#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "kernel_ir.h"

namespace mlk::hip {

enum class StepKind : uint8_t { Elementwise, Softmax, Gemm, RowSum, ScoreSoftmax, Nest, Fail };

/// One read or write of a buffer over an R-dim box: element (v0..vR-1),
/// v_d in [0, extent_d), touches buffer[offset + sum coeff[d] * v_d].
struct StreamRef {
    uint32_t buffer{kInvalidId};
    int64_t offset{0};
    int64_t coeff[4]{0, 0, 0, 0};
};

/// Elements of one row segment of the elementwise template (one wave: 64
/// lanes x 8 elements); the grid has one wave per segment.
constexpr int64_t kElementwiseSegment = 512;

struct Step {
    StepKind kind{StepKind::Fail};
    std::string what;                 // class name for reports

    // Elementwise (JIT instance of elementwise_template.hip).
    int rank{1};
    int64_t extent[4]{1, 1, 1, 1};
    bool dynamicExtent{false};        // 1-D loop bound = io.elements
    int64_t dynBegin{0};              // dynamic form: first index
    std::vector<StreamRef> inputs;
    StreamRef out;
    AccumMode accum{AccumMode::None};
    std::string chainBody;
    /// The chain in the reference's f64 forms when chainBody uses a form that
    /// can decline an element (split-precision sin, f32-accurate exp); empty
    /// otherwise.
    std::string chainExact;
    std::string source;
    std::string kernelName;           // hipRTC symbol (elementwise and nest steps)
    void* fn{nullptr};

    // Softmax / RowSum: rows x cols from buffer x into y.
    uint32_t x{kInvalidId}, y{kInvalidId};
    int64_t rows{0}, cols{0};

    // Gemm: C[M,N] (+)= A[M,K] B[K,N] (batched with per-batch strides).
    uint32_t a{kInvalidId}, b{kInvalidId}, c{kInvalidId};
    int64_t m{0}, n{0}, k{0};
    int64_t lda{0}, ldb{0}, ldc{0};
    bool accumulate{false};
    // Call(MatMul) skips A[i,p] == 0 (gemmRowBlock, kernel_buffers.cpp:422):
    // before the launch B is scanned for non-finite values, and when it holds
    // any the exact general kernel with the skip runs instead of the MFMA
    // forms (0 * inf would make NaN where the reference adds nothing).
    bool skipZeroA{false};

    // ScoreSoftmax: S = softmax(Q K^T / div + bias) per batch.
    uint32_t q{kInvalidId}, kk{kInvalidId}, bias{kInvalidId}, s{kInvalidId};
    int64_t batch{0}, seq{0}, dim{0};
    double div{1.0};

    // Nest (generic loop nest, nestgen.cpp): one forest root as a hipRTC
    // kernel; `nestBufs` maps kernel buffer slots to buffer ids; `threads` is
    // the padded instance count of the collapsed parallel loops; `checked`
    // means some access carries a run-time bounds check whose status word is
    // read back after the launch.
    uint32_t root{kInvalidId};
    // LDS slabs of the nest kernel, and the same kernel without them (empty
    // when it has none): launch form 1 of the step, compiled on first use.
    int slabs{0};
    std::string sourceNoSlabs;
    // Launch form 4: the innermost collapsed loop run inside each thread
    // (empty when not declared), its instance count and bounds-check flag.
    std::string sourceLessCollapse;
    int64_t threadsLessCollapse{0};
    bool checkedLessCollapse{false};
    std::vector<uint32_t> nestBufs;
    std::vector<uint32_t> nestWrites;
    std::vector<uint32_t> nestReads;  // buffers the kernel reads from memory (registers' loads included)
    // Element hulls of the step's reads and writes per buffer id (lo > hi:
    // none); empty vectors mean whole buffers.
    std::vector<std::pair<int64_t, int64_t>> readHull, writeHull;
    int64_t threads{0};
    int collapsed{0};
    bool checked{false};
    bool transcendental{false};
    bool narrowRoundTrip{false};
    bool touchesF16{false};

    // Launch form of a hand-written kernel (-1: the kernel's default); set
    // by mlkhip_set_step_variant, the variant search or its cache.
    int variant{-1};

    // Fail: the step reports this ABI code at run time (1 = negative store
    // address, as the reference walker's InvalidGraph at execution).
    int failCode{0};
};

struct Plan {
    std::string className;            // joined step classes
    std::string policy;               // tolerance policy id
    bool multiDim{false};
    bool canonicalized{false};        // planned on canonicalModule's rewrite
    std::vector<Step> steps;
    std::vector<bool> tempNeeded;     // per buffer id: device scratch needed
};

/// Recognizes every root of `km` (or every top-level node of a 1-D module)
/// as a supported class. Refuses honestly (UnsupportedCapability) what no
/// hand-written kernel covers.
Result<Plan> planModule(const KernelModule& km);

/// Full hipRTC source of an elementwise step (prelude + template); its
/// kernel symbol, mlk_elementwise_<12 hex digits of the source's FNV-1a>, goes
/// to `kernelName` when given.
std::string elementwiseSource(const KernelModule& km, const Step& st, std::string* kernelName = nullptr);

/// The device math header text every hipRTC instance starts with.
const char* deviceMathHeader();

/// The module as the device holds it: temps in f64, as the reference
/// executor holds every buffer (kernel_buffers.cpp:852-878).
KernelModule deviceModule(const KernelModule& km);

/// Canonical form of a multi-dim module (canonical.cpp): poly.codegen's
/// strip-mined, split and guarded bands rewritten to their untiled loop
/// forms where the rewrite keeps the walker's order exactly. `rewrites` is
/// set to 1 when anything changed. Buffers are unchanged.
KernelModule canonicalModule(const KernelModule& km, int* rewrites);

/// Generic loop-nest step for one forest root (nestgen.cpp): the root's
/// subtree as straight-line f64 device code, the outermost parallel loops
/// collapsed onto threads. The step's `source` holds the hipRTC text.
Result<Step> planNest(const KernelModule& km, uint32_t root);

/// Launch forms of a loop-nest step (nestgen.cpp): 0 the step's own kernel
/// (its LDS slabs, 256 threads per workgroup); 1 the same kernel without
/// slabs (declared only where the step has slabs); 2 and 3 form 0 with 512
/// and 64 threads per workgroup; 4 the kernel with its innermost collapsed
/// loop run inside each thread (declared where two or more loops collapse
/// and both forms keep the walker's values). Every form computes each
/// instance with the same operations, so all give the same bits.
std::vector<int> nestForms(const Step& st);
/// Instances (threads' work items) and the bounds-check flag of form `form`.
int64_t nestFormInstances(const Step& st, int form);
bool nestFormChecked(const Step& st, int form);
/// Threads per workgroup of loop-nest form `form`.
unsigned nestFormThreads(int form);
/// hipRTC source of loop-nest form `form` of `st` (empty if not declared).
std::string nestFormSource(const Step& st, int form);

/// Hex-float literal of an f64 constant (exact), or the non-finite builtins.
std::string literal(double v);

/// f64 chain body (kernel_buffers.cpp:106-178 semantics). `elemCode` gives the
/// device expression of an ElemIdx/ElemA/ElemB operand ("" = unrealizable);
/// the result is written as `<sink>tN;`.
Result<std::string> chainCode(const std::vector<KernelExpr>& exprs, bool poly7, bool f32Out,
                              const std::function<std::string(const KernelOperand&)>& elemCode,
                              const std::string& sink,
                              const std::function<int(const KernelOperand&)>& elemBits = {});

/// Buffer element count as the executors size it (dims product, else
/// `elements`; dynamic buffers take the run's element count).
int64_t bufferElements(const KernelBuffer& b, int64_t dynamicElements);

}  // namespace mlk::hip
