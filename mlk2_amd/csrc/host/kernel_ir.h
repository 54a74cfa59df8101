// Kernel IR as the HIP backend consumes it: a restatement of
// compiler/include/mlk/support/kernel_ir.h:22-224 (KernelOp, AccumMode,
// KernelOperand, KernelExpr, KernelNode, KernelBuffer, KernelModule) with
// plain std::vector storage, plus the reader for the "mlk-kernel" document
// KernelModule::toJson writes (compiler/src/support/kernel_ir.cpp:97-254).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "expected.h"

namespace mlk::hip {

inline constexpr uint32_t kInvalidId = 0xFFFFFFFFu;                  // constants.h:15
inline constexpr int64_t kDynamicBound = -1;                         // constants.h:92
inline constexpr int64_t kTempElementsLimit = int64_t{1} << 24;      // constants.h:99
inline constexpr int64_t kDefaultTileM = 64, kDefaultTileN = 64, kDefaultTileK = 32;  // constants.h:84-86

enum class KernelOp : uint8_t { Loop, Compute, Load, Store, AllocBuffer, CopyBuffer, Barrier, Trace, Guard, Call };

/// MathOp subset the Kernel IR carries (compiler/include/mlk/ir/math_op.h:18-79).
enum class MathOp : uint8_t {
    Add, Sub, Mul, Div, Neg, Pow, Exp, Log, Sin, Cos, Tan, Tanh, Sqrt, Rsqrt, Erf, Gelu,
    MatMul, ReduceSum, Softmax, Other
};

enum class AccumMode : uint8_t { None, Add, Max };
enum class Dtype : uint8_t { F32, F16, F64, Other };

struct KernelOperand {
    enum class Kind : uint8_t { Const, ElemA, ElemB, ScalarParam, Temp, ElemIdx };
    Kind kind{Kind::Const};
    int64_t index{0};
    double constValue{0.0};
    std::vector<int64_t> idxCoeffs;
    int64_t idxOffset{0};
};

struct KernelExpr {
    MathOp op{MathOp::Add};
    KernelOperand a, b;
};

struct KernelNode {
    KernelOp op{KernelOp::Loop};
    MathOp math{MathOp::Add};
    std::string var;
    int64_t begin{0};
    int64_t end{kDynamicBound};
    int64_t step{1};
    std::vector<int64_t> beginCoeffs;
    int64_t beginOffset{0};
    std::vector<int64_t> endCoeffs;
    int64_t endOffset{0};
    uint32_t endBuf{kInvalidId};
    int32_t endDim{-1};
    uint32_t bufferA{kInvalidId}, bufferB{kInvalidId}, bufferOut{kInvalidId};
    std::vector<int64_t> outIndexCoeffs;
    int64_t outIndexOffset{0};
    AccumMode accum{AccumMode::None};
    bool parallel{false};
    bool vectorHint{false};
    std::vector<int64_t> guardCoeffs;
    int64_t guardOffset{0};
    std::string family;
    std::vector<KernelExpr> exprs;
    std::vector<uint32_t> children;

    bool hasAffineStore() const { return !outIndexCoeffs.empty(); }
    bool hasAffineGuard() const { return !guardCoeffs.empty(); }
};

struct KernelBuffer {
    std::string name;
    Dtype dtype{Dtype::F32};
    bool isInput{false}, isOutput{false}, isTemp{false};
    int64_t elements{kDynamicBound};
    std::vector<int64_t> dims;
};

struct KernelModule {
    std::vector<KernelBuffer> buffers;
    std::vector<KernelNode> nodes;
    std::string name;
    std::vector<std::pair<std::string, int64_t>> schedule;

    int64_t param(const char* key, int64_t fallback) const {
        for (const auto& kv : schedule) {
            if (kv.first == key) return kv.second;
        }
        return fallback;
    }
};

/// Parses an "mlk-kernel" document. Accepts the reference writer's output
/// and two extensions: "math" on Call nodes, and Infinity/-Infinity/NaN
/// tokens for exact non-finite constants.
Result<KernelModule> parseKernelModule(const char* text, size_t len);

/// Same multi-dim test as the reference executor (kernel_buffers.cpp:883-901)
/// and backends/cpu/src/cpp_emitter.cpp:667-687: any ElemIdx operand, affine
/// bound, accumulate store, buffer-dim bound, affine store or affine guard.
bool isMultiDimModule(const KernelModule& km);

/// Forest roots in id order (nodes no other node lists as a child).
std::vector<uint32_t> forestRoots(const KernelModule& km);

int dtypeBytes(Dtype d);
const char* mathOpName(MathOp op);
bool isUnaryMath(MathOp op);

/// 64-bit structural hash of the module (the role of KernelModule::hash,
/// kernel_ir.cpp:37-95): every field that changes execution semantics.
uint64_t moduleHash(const KernelModule& km);

}  // namespace mlk::hip
