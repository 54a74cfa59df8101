"""Host-side mirror of the reference Kernel IR data model.

Restates ``compiler/include/mlk/support/kernel_ir.h:22-224`` (KernelOp,
AccumMode, KernelOperand, KernelExpr, KernelNode, KernelBuffer, KernelModule)
as plain Python objects, and serializes them to the "mlk-kernel" JSON document
that ``KernelModule::toJson`` writes (``compiler/src/support/kernel_ir.cpp:97-254``).
That document is the module interchange of the HIP backend's C ABI.

``to_json`` writes two extensions of the reference writer that carry a module
losslessly: Call nodes carry ``"math"`` (the reference writer emits it for
Compute nodes only), and non-finite constants are written as the tokens
``Infinity`` / ``-Infinity`` / ``NaN`` (the reference writer clamps +/-inf to
+/-1e308 and NaN to null, ``compiler/src/core/json.cpp:300-312``).
``to_reference_json`` writes the reference writer's own document, which the
backend's reader takes unchanged: it infers a Call's target from its operands
and reads +/-1e308 back as +/-inf.
"""
from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from typing import List, Optional

INVALID_ID = 0xFFFFFFFF          # constants::kInvalidId (constants.h:15)
DYNAMIC = -1                     # constants::kKernelLoopDynamicBound (constants.h:92)
TEMP_ELEMENTS_LIMIT = 1 << 24    # constants::kKernelTempElementsLimit (constants.h:99)

# MathOp names as printed by the reference op table (compiler/src/ir/math_op.cpp:16-45).
UNARY_OPS = {"neg", "exp", "log", "sin", "cos", "tan", "tanh", "sqrt", "rsqrt",
             "erf", "gelu"}
SCALAR_OPS = {"add", "sub", "mul", "div", "pow"} | UNARY_OPS


@dataclass
class KernelOperand:
    """kernel_ir.h:58-83. kind is one of const, elem_a, elem_b, scalar_param,
    temp, elem_idx."""
    kind: str = "const"
    index: int = 0
    value: float = 0.0
    coeffs: List[int] = field(default_factory=list)
    offset: int = 0

    def to_json(self) -> dict:
        o = {"kind": self.kind}
        if self.kind == "const":
            o["value"] = float(self.value)
        if self.kind in ("temp", "scalar_param"):
            o["index"] = int(self.index)
        if self.kind == "elem_idx":
            o["buffer"] = int(self.index)
            o["coeffs"] = [int(c) for c in self.coeffs]
            o["offset"] = int(self.offset)
        return o


def const(v: float) -> KernelOperand:
    return KernelOperand("const", value=v)


def elem_a() -> KernelOperand:
    return KernelOperand("elem_a")


def elem_b() -> KernelOperand:
    return KernelOperand("elem_b")


def scalar(i: int) -> KernelOperand:
    return KernelOperand("scalar_param", index=i)


def temp(i: int) -> KernelOperand:
    return KernelOperand("temp", index=i)


def elem_idx(buf: int, coeffs, offset: int = 0) -> KernelOperand:
    return KernelOperand("elem_idx", index=buf, coeffs=list(coeffs), offset=offset)


@dataclass
class KernelExpr:
    """kernel_ir.h:89-97: one SSA op of a fused Compute chain."""
    op: str = "add"
    a: KernelOperand = field(default_factory=KernelOperand)
    b: KernelOperand = field(default_factory=KernelOperand)

    def to_json(self) -> dict:
        return {"op": self.op, "a": self.a.to_json(), "b": self.b.to_json()}


@dataclass
class KernelNode:
    """kernel_ir.h:99-174."""
    op: str = "loop"                 # loop compute load store alloc copy barrier trace guard call
    math: str = "add"
    var: Optional[str] = None
    begin: int = 0
    end: int = DYNAMIC
    step: int = 1
    begin_coeffs: List[int] = field(default_factory=list)
    begin_offset: int = 0
    end_coeffs: List[int] = field(default_factory=list)
    end_offset: int = 0
    end_buf: int = INVALID_ID
    end_dim: int = -1
    a: int = INVALID_ID
    b: int = INVALID_ID
    out: int = INVALID_ID
    out_index_coeffs: List[int] = field(default_factory=list)
    out_index_offset: int = 0
    accum: str = "none"              # none | add | max  (AccumMode, kernel_ir.h:43-47)
    parallel: bool = False
    vector_hint: bool = False
    guard_coeffs: List[int] = field(default_factory=list)
    guard_offset: int = 0
    family: Optional[str] = None
    exprs: List[KernelExpr] = field(default_factory=list)
    children: List[int] = field(default_factory=list)

    def to_json(self) -> dict:
        o = {"op": self.op}
        if self.op in ("compute", "call"):
            o["math"] = self.math
            if self.family is not None:
                o["family"] = self.family
        if self.var is not None:
            o["var"] = self.var
        o["begin"] = int(self.begin)
        o["end"] = int(self.end)
        o["step"] = int(self.step)
        if self.end_buf != INVALID_ID:
            o["end_buf"] = int(self.end_buf)
            o["end_dim"] = int(self.end_dim)
        if self.begin_coeffs or self.end_coeffs:
            o["begin_coeffs"] = [int(c) for c in self.begin_coeffs]
            o["begin_offset"] = int(self.begin_offset)
            o["end_coeffs"] = [int(c) for c in self.end_coeffs]
            o["end_offset"] = int(self.end_offset)
        if self.out_index_coeffs:
            o["out_index_coeffs"] = [int(c) for c in self.out_index_coeffs]
            o["out_index_offset"] = int(self.out_index_offset)
            if self.accum != "none":
                o["accumulate"] = True
                if self.accum == "max":
                    o["accum_mode"] = "max"
        if self.op == "loop" and self.parallel:
            o["parallel"] = True
        if self.op == "loop" and self.vector_hint:
            o["vector_hint"] = True
        if self.op == "guard" and self.guard_coeffs:
            o["guard_coeffs"] = [int(c) for c in self.guard_coeffs]
            o["guard_offset"] = int(self.guard_offset)
        if self.a != INVALID_ID:
            o["a"] = int(self.a)
        if self.b != INVALID_ID:
            o["b"] = int(self.b)
        if self.out != INVALID_ID:
            o["out"] = int(self.out)
        if self.exprs:
            o["exprs"] = [e.to_json() for e in self.exprs]
        o["children"] = [int(c) for c in self.children]
        return o


@dataclass
class KernelBuffer:
    """kernel_ir.h:176-194."""
    name: str = "buf"
    dtype: str = "f32"
    is_input: bool = False
    is_output: bool = False
    is_temp: bool = False
    elements: int = DYNAMIC
    dims: List[int] = field(default_factory=list)

    def to_json(self) -> dict:
        o = {"name": self.name, "dtype": self.dtype, "input": self.is_input,
             "output": self.is_output}
        if self.is_temp:
            o["temp"] = True
        o["elements"] = int(self.elements)
        if self.dims:
            o["dims"] = [int(d) for d in self.dims]
        return o


@dataclass
class KernelModule:
    """kernel_ir.h:196-217."""
    buffers: List[KernelBuffer] = field(default_factory=list)
    nodes: List[KernelNode] = field(default_factory=list)
    name: str = "mlk_kernel"
    schedule: dict = field(default_factory=dict)

    def add_buffer(self, b: KernelBuffer) -> int:
        self.buffers.append(b)
        return len(self.buffers) - 1

    def add_node(self, n: KernelNode) -> int:
        self.nodes.append(n)
        return len(self.nodes) - 1

    def to_dict(self) -> dict:
        return {
            "format": "mlk-kernel",
            "version": 1,
            "name": self.name,
            "buffers": [b.to_json() for b in self.buffers],
            "nodes": [n.to_json() for n in self.nodes],
            "schedule": {k: int(v) for k, v in self.schedule.items()},
        }

    def to_json(self) -> str:
        # allow_nan=True writes Infinity/-Infinity/NaN tokens for exact
        # non-finite constants (see module docstring).
        return json.dumps(self.to_dict(), separators=(",", ":"), allow_nan=True)

    def to_reference_json(self) -> str:
        """The document exactly as the reference's writer produces it
        (``KernelModule::toJson``, ``compiler/src/support/kernel_ir.cpp:97-254``,
        serialized by ``compiler/src/core/json.cpp:301-312``): ``"math"`` and
        ``"family"`` only on Compute nodes, +/-inf constants clamped to
        +/-1e308, NaN written as null, doubles printed with 17 significant
        digits. The backend's reader accepts it unchanged: a Call's target is
        inferred from its operands and +/-1e308 reads back as +/-inf."""
        d = self.to_dict()
        for n in d["nodes"]:
            if n["op"] != "compute":
                n.pop("math", None)
                n.pop("family", None)
        return _reference_serialize(d)

    # --- binding helpers (KernelBufferBindings layout, execution.h:117-130)
    def input_ids(self) -> List[int]:
        return [i for i, b in enumerate(self.buffers) if b.is_input]

    def output_ids(self) -> List[int]:
        return [i for i, b in enumerate(self.buffers) if b.is_output]

    def bindable_ids(self) -> List[int]:
        """Buffer-table ids bound through the artifact ABI: input | output |
        temp, in table order (backend_driver.h:15-46)."""
        return [i for i, b in enumerate(self.buffers)
                if b.is_input or b.is_output or b.is_temp]

    def roots(self) -> List[int]:
        referenced = set()
        for n in self.nodes:
            referenced.update(n.children)
        return [i for i in range(len(self.nodes)) if i not in referenced]


def is_multidim_module(km: KernelModule) -> bool:
    """isMultiDimModule (backends/cpu/src/cpp_emitter.cpp:667-687): selects
    the artifact ABI form (multi-dim int return vs legacy 1-D void)."""
    for n in km.nodes:
        if n.accum != "none" or n.begin_coeffs or n.end_coeffs or n.out_index_coeffs:
            return True
        if n.end == DYNAMIC and n.end_buf != INVALID_ID:
            return True
        if n.op == "guard" and n.guard_coeffs:
            return True
        for e in n.exprs:
            if e.a.kind == "elem_idx" or e.b.kind == "elem_idx":
                return True
    return False


def is_finite_const(v: float) -> bool:
    return math.isfinite(v)


def _reference_double(v: float) -> str:
    """serializeDouble (compiler/src/core/json.cpp:301-312)."""
    if math.isnan(v):
        return "null"
    if math.isinf(v):
        return "1e308" if v > 0 else "-1e308"
    return "%.17g" % v


def _reference_serialize(v) -> str:
    if v is True:
        return "true"
    if v is False:
        return "false"
    if v is None:
        return "null"
    if isinstance(v, int):
        return str(v)
    if isinstance(v, float):
        return _reference_double(v)
    if isinstance(v, str):
        return json.dumps(v)
    if isinstance(v, list):
        return "[" + ",".join(_reference_serialize(x) for x in v) + "]"
    return "{" + ",".join(json.dumps(k) + ":" + _reference_serialize(x) for k, x in v.items()) + "}"
