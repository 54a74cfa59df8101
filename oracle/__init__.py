"""ctypes loader for the CPU oracle (oracle/oracle.cpp) — test infrastructure.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker; the product library never does.
"""
from __future__ import annotations

import ctypes
import os
from typing import Dict, List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "liboracle.so")
REF_PATH = os.path.join(_HERE, "_ref", "libref_families.so")

_lib = None
_ref = None

_PD = ctypes.POINTER(ctypes.c_double)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_execute.restype = ctypes.c_int
        L.oracle_execute.argtypes = [ctypes.c_char_p, ctypes.c_size_t,
                                     ctypes.POINTER(_PD), ctypes.c_int,
                                     ctypes.POINTER(_PD), ctypes.c_int,
                                     _PD, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                     ctypes.c_char_p, ctypes.c_size_t]
        L.oracle_poly_sin.restype = ctypes.c_double
        L.oracle_poly_sin.argtypes = [ctypes.c_double]
        L.oracle_poly_sin_many.restype = None
        L.oracle_poly_sin_many.argtypes = [_PD, _PD, ctypes.c_int64]
        L.oracle_gemm_blocked.restype = None
        L.oracle_gemm_blocked.argtypes = [_PD, _PD, _PD] + [ctypes.c_int64] * 6
        _lib = L
    return _lib


def ref_lib():
    """The reference's own math_families.h compiled into oracle/_ref, or None
    where it was not built (no reference tree)."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        L = ctypes.CDLL(REF_PATH)
        L.ref_poly_sin.restype = ctypes.c_double
        L.ref_poly_sin.argtypes = [ctypes.c_double]
        L.ref_measured_poly_sin_max_ulps.restype = ctypes.c_double
        L.ref_measured_poly_sin_max_ulps.argtypes = []
        _ref = L
    return _ref


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_PD)


class OracleError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"oracle error {code}: {msg}")
        self.code = code
        self.msg = msg


def execute(km_json: str, inputs: Sequence[np.ndarray], outputs: Sequence[np.ndarray],
            scalars: Sequence[float] = (), elements: int = 0, hw_threads: int = 1) -> None:
    """Runs the module over f64 buffers in place (reference binding rules:
    ``inputs`` in input-buffer order, ``outputs`` in output order)."""
    for a in list(inputs) + list(outputs):
        assert a.dtype == np.float64 and a.flags.c_contiguous
    ins = (_PD * max(1, len(inputs)))(*[_ptr(a) for a in inputs])
    outs = (_PD * max(1, len(outputs)))(*[_ptr(a) for a in outputs])
    sc = np.ascontiguousarray(np.asarray(scalars, dtype=np.float64).reshape(-1))
    if sc.size == 0:
        sc = np.zeros(1)
        nsc = 0
    else:
        nsc = sc.size
    msg = ctypes.create_string_buffer(512)
    data = km_json.encode()
    rc = lib().oracle_execute(data, len(data), ins, len(inputs), outs, len(outputs),
                              _ptr(sc), nsc, int(elements), int(hw_threads), msg, 512)
    if rc != 0:
        raise OracleError(rc, msg.value.decode())


def run(km, arrays: Dict[int, np.ndarray], scalars: Sequence[float] = (),
        elements: int = 0, hw_threads: int = 1, init: Optional[Dict[int, np.ndarray]] = None
        ) -> Dict[int, np.ndarray]:
    """Convenience: ``arrays`` maps input buffer ids to arrays (any float
    dtype; widened exactly to f64). Outputs start at zero (or ``init``) and
    are returned by buffer id as f64."""
    ins: List[np.ndarray] = []
    for bid in km.input_ids():
        ins.append(np.ascontiguousarray(np.asarray(arrays[bid], dtype=np.float64).reshape(-1)))
    outs: List[np.ndarray] = []
    for bid in km.output_ids():
        b = km.buffers[bid]
        n = b.elements if b.elements > 0 else int(elements)
        if init is not None and bid in init:
            outs.append(np.array(init[bid], dtype=np.float64).reshape(-1))  # a copy: init is not written
        else:
            outs.append(np.zeros(n, dtype=np.float64))
    execute(km.to_json(), ins, outs, scalars, elements, hw_threads)
    return {bid: o for bid, o in zip(km.output_ids(), outs)}


def poly_sin(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(x)
    lib().oracle_poly_sin_many(_ptr(x), _ptr(y), x.size)
    return y
