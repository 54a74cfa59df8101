"""Python host interface over libmlk_hip.so (include/mlk_hip.h).

Mirrors the reference's driver surface (backends/cpu/include/mlk/backend/
backend_driver.h:91-228): ``HipBackendDriverConfig`` / ``build_hip_kernel_artifact``
/ ``LoadedKernel.run`` over the f64 host ABI, plus the device-resident typed
entry used for timing. Every call goes through the C ABI; there is no Python
or CPU fallback: a missing library or device raises.
"""
from __future__ import annotations

import ctypes
import json
import os
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import numpy as np

from .kernel_ir import KernelModule

HERE = os.path.dirname(os.path.abspath(__file__))
# MLK_HIP_LIB names another build of the same library (the host-sanitized
# one that tests/test_host_sanitizers.py links); by default the in-tree one.
LIB_PATH = os.environ.get("MLK_HIP_LIB") or os.path.join(HERE, "lib", "libmlk_hip.so")

OK, NEG_STORE, RUNTIME, LAUNCH, NO_DEVICE, BAD_BINDING, REFUSED = 0, 1, 2, 3, 4, 6, 7
F32, F16, F64 = 0, 1, 2
DTYPE_CODE = {"f32": F32, "f16": F16, "f64": F64}
NP_OF_CODE = {F32: np.float32, F16: np.float16, F64: np.float64}

_PD = ctypes.POINTER(ctypes.c_double)


class MlkHipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"mlk_hip status {code}: {message}")
        self.code = code
        self.message = message


class Binding(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("elements", ctypes.c_int64),
                ("dtype", ctypes.c_int32), ("pad", ctypes.c_int32)]


_lib = None


def lib():
    """Loads libmlk_hip.so (built in-tree by __graft_entry__.build())."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    c = ctypes
    L.mlkhip_last_error.restype = c.c_char_p
    L.mlkhip_device_available.argtypes = [c.c_char_p]
    L.mlkhip_valid_arch.argtypes = [c.c_char_p]
    L.mlkhip_build.argtypes = [c.c_char_p, c.c_size_t, c.c_char_p, c.c_char_p, c.POINTER(c.c_void_p)]
    L.mlkhip_plan.argtypes = [c.c_char_p, c.c_size_t, c.c_char_p, c.c_size_t, c.c_char_p,
                              c.c_size_t, c.POINTER(c.c_int)]
    L.mlkhip_compile_check.restype = c.c_longlong
    L.mlkhip_compile_check.argtypes = [c.c_char_p, c.c_size_t, c.c_int, c.c_char_p, c.c_char_p,
                                       c.c_size_t]
    L.mlkhip_release.argtypes = [c.c_void_p]
    L.mlkhip_release.restype = None
    L.mlkhip_release_stream_scratch.argtypes = [c.c_void_p, c.c_void_p]
    L.mlkhip_is_multidim.argtypes = [c.c_void_p]
    L.mlkhip_class_name.argtypes = [c.c_void_p]
    L.mlkhip_class_name.restype = c.c_char_p
    L.mlkhip_policy.argtypes = [c.c_void_p]
    L.mlkhip_policy.restype = c.c_char_p
    L.mlkhip_num_bindables.argtypes = [c.c_void_p]
    L.mlkhip_bindable_info.argtypes = [c.c_void_p, c.c_int, c.POINTER(c.c_int32),
                                       c.POINTER(c.c_int64), c.POINTER(c.c_int),
                                       c.POINTER(c.c_int), c.POINTER(c.c_int)]
    L.mlkhip_kernel.argtypes = [c.c_void_p, c.POINTER(_PD), c.POINTER(c.POINTER(c.c_int64)),
                                c.c_int, _PD, c.c_int64, c.c_int64]
    L.mlkhip_kernel_1d.argtypes = [c.c_void_p, c.POINTER(_PD), c.c_int, c.c_int64, _PD, c.c_int64]
    L.mlkhip_run_device.argtypes = [c.c_void_p, c.POINTER(Binding), c.c_int, _PD, c.c_int64,
                                    c.c_int64, c.c_void_p]
    L.mlkhip_time_device.argtypes = [c.c_void_p, c.POINTER(Binding), c.c_int, _PD, c.c_int64,
                                     c.c_int64, c.c_void_p, c.c_int, c.c_int,
                                     c.POINTER(c.c_float)]
    L.mlkhip_time_device_span.argtypes = [c.c_void_p, c.POINTER(Binding), c.c_int, _PD, c.c_int64,
                                          c.c_int64, c.c_void_p, c.c_int, c.c_int,
                                          c.POINTER(c.c_float)]
    L.mlkhip_num_steps.argtypes = [c.c_void_p]
    L.mlkhip_step_variants.argtypes = [c.c_void_p, c.c_int, c.POINTER(c.c_int), c.c_int]
    L.mlkhip_plan_variants.argtypes = [c.c_char_p, c.c_size_t, c.c_int, c.POINTER(c.c_int), c.c_int]
    L.mlkhip_step_variant.argtypes = [c.c_void_p, c.c_int]
    L.mlkhip_set_step_variant.argtypes = [c.c_void_p, c.c_int, c.c_int]
    L.mlkhip_fingerprint.argtypes = [c.c_void_p]
    L.mlkhip_fingerprint.restype = c.c_char_p
    L.mlkhip_variants_from_cache.argtypes = [c.c_void_p]
    L.mlkhip_autotune.argtypes = [c.c_void_p, c.POINTER(Binding), c.c_int, _PD, c.c_int64, c.c_int64,
                                  c.c_int, c.c_char_p, c.c_char_p, c.c_size_t]
    L.mlkhip_essential_work.argtypes = [c.c_char_p, c.c_size_t, c.c_double, c.c_double, c.POINTER(c.c_int64),
                                        c.POINTER(c.c_int64), c.POINTER(c.c_int), c.POINTER(c.c_int),
                                        c.POINTER(c.c_double)]
    L.mlkhip_measure_environment.argtypes = [c.POINTER(c.c_double), c.POINTER(c.c_double)]
    L.mlkhip_execute_kernel_on_buffers.argtypes = [c.c_char_p, c.c_size_t, c.c_char_p, c.POINTER(_PD), c.c_int,
                                                   c.POINTER(_PD), c.c_int, _PD, c.c_int64, c.c_int64]
    L.mlkhip_execute_kernel.argtypes = [c.c_char_p, c.c_size_t, c.c_char_p, _PD, c.c_int, _PD, c.c_int]
    L.mlkhip_execute_cache_size.argtypes = []
    L.mlkhip_execute_cache_clear.argtypes = []
    L.mlkhip_execute_cache_clear.restype = None
    L.mlkhip_malloc.argtypes = [c.POINTER(c.c_void_p), c.c_size_t]
    L.mlkhip_free.argtypes = [c.c_void_p]
    L.mlkhip_memcpy_h2d.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t]
    L.mlkhip_memcpy_d2h.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t]
    L.mlkhip_fill32.argtypes = [c.c_void_p, c.c_uint32, c.c_size_t]
    L.mlkhip_stream_create.argtypes = [c.POINTER(c.c_void_p)]
    L.mlkhip_stream_destroy.argtypes = [c.c_void_p]
    L.mlkhip_run_device_noalloc.argtypes = [c.c_void_p, c.POINTER(Binding), c.c_int, _PD, c.c_int64,
                                            c.c_int64, c.c_void_p]
    L.mlkhip_noalloc_scratch_bytes.argtypes = []
    L.mlkhip_noalloc_scratch_bytes.restype = c.c_size_t
    L.mlkhip_emit_artifact.argtypes = [c.c_char_p, c.c_size_t, c.c_char_p, c.c_char_p, c.c_char_p, c.c_char_p,
                                       c.c_size_t]
    L.mlkhip_jit_options.argtypes = [c.c_char_p, c.c_char_p, c.c_size_t]
    L.mlkhip_step_kernel_name.argtypes = [c.c_void_p, c.c_int]
    L.mlkhip_step_kernel_name.restype = c.c_char_p
    _lib = L
    return L


def last_error() -> str:
    return lib().mlkhip_last_error().decode(errors="replace")


def _check(rc: int) -> None:
    if rc != OK:
        raise MlkHipError(rc, last_error())


@dataclass
class HipBackendDriverConfig:
    """GpuBackendDriverConfig analogue (backend_driver.h:91-105): the target
    is declared, never defaulted from the device."""
    arch: str = "gfx950"
    cache_dir: Optional[str] = None


def plan(km: KernelModule):
    """(class name, policy, steps) without compiling or loading."""
    data = km.to_json().encode()
    cls = ctypes.create_string_buffer(512)
    pol = ctypes.create_string_buffer(128)
    n = ctypes.c_int(0)
    _check(lib().mlkhip_plan(data, len(data), cls, 512, pol, 128, ctypes.byref(n)))
    return cls.value.decode(), pol.value.decode(), n.value


def compile_check(km: KernelModule, step: int = 0, arch: str = "gfx950"):
    """Instantiates step `step`'s template and compiles it with hipRTC (no
    device needed). Returns (code-object bytes, source)."""
    data = km.to_json().encode()
    src = ctypes.create_string_buffer(1 << 20)
    n = lib().mlkhip_compile_check(data, len(data), step, arch.encode(), src, 1 << 20)
    if n < 0:
        raise MlkHipError(REFUSED, last_error())
    return n, src.value.decode()


def plan_variants(km: KernelModule, step: int = 0) -> List[int]:
    """Declared launch forms of step `step` (first = default; empty when the
    step has only its default form), without a device."""
    data = km.to_json().encode()
    out = (ctypes.c_int * 32)()
    n = lib().mlkhip_plan_variants(data, len(data), step, out, 32)
    if n < 0:
        raise MlkHipError(REFUSED, last_error())
    return list(out[:n])


def essential_work(km: KernelModule, bytes_per_sec: float = 0.0, ops_per_sec: float = 0.0) -> dict:
    """EssentialWork + roofline lower bound (mlkhip_essential_work); rates
    <= 0 take the MI355X datasheet values. No device needed."""
    data = km.to_json().encode()
    b, o = ctypes.c_int64(), ctypes.c_int64()
    bk, ok = ctypes.c_int(), ctypes.c_int()
    low = ctypes.c_double()
    _check(lib().mlkhip_essential_work(data, len(data), float(bytes_per_sec), float(ops_per_sec), ctypes.byref(b),
                                       ctypes.byref(o), ctypes.byref(bk), ctypes.byref(ok), ctypes.byref(low)))
    return {"min_bytes": b.value, "min_ops": o.value, "bytes_known": bool(bk.value), "ops_known": bool(ok.value),
            "roofline_lower_sec": low.value}


def measure_environment() -> dict:
    """Measured HBM bytes/s and f16 MFMA flop/s of the device (probed once)."""
    bw, f16 = ctypes.c_double(), ctypes.c_double()
    _check(lib().mlkhip_measure_environment(ctypes.byref(bw), ctypes.byref(f16)))
    return {"bytes_per_sec": bw.value, "f16_flops_per_sec": f16.value}


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64).reshape(-1))


def execute_kernel_on_buffers(km: KernelModule, inputs: Sequence[np.ndarray], outputs: Sequence[np.ndarray],
                              scalars: Sequence[float] = (), elements: int = 0, arch: str = "gfx950") -> None:
    """executeKernelOnBuffers analogue (the run route): dense f64 host arrays,
    inputs in input-buffer order, outputs in output-buffer order; each output
    must be a C-contiguous float64 array and is updated in place."""
    for o in outputs:
        if not (isinstance(o, np.ndarray) and o.dtype == np.float64 and o.flags.c_contiguous):
            raise MlkHipError(BAD_BINDING, "outputs must be C-contiguous float64 arrays")
    ins = [_f64(a) for a in inputs]
    data = km.to_json().encode()
    pin = (_PD * max(1, len(ins)))(*[a.ctypes.data_as(_PD) for a in ins])
    pout = (_PD * max(1, len(outputs)))(*[o.ctypes.data_as(_PD) for o in outputs])
    sc = np.asarray(list(scalars) or [0.0], dtype=np.float64)
    _check(lib().mlkhip_execute_kernel_on_buffers(data, len(data), arch.encode(), pin, len(ins), pout,
                                                  len(outputs), sc.ctypes.data_as(_PD), len(scalars),
                                                  int(elements)))


def execute_kernel(km: KernelModule, input_scalars: Sequence[float], arch: str = "gfx950") -> List[float]:
    """executeKernel analogue (scalar ABI): ScalarParams in, element 0 of
    each output buffer out."""
    data = km.to_json().encode()
    n_out = sum(1 for b in km.buffers if b.is_output)
    out = np.zeros(max(1, n_out), dtype=np.float64)
    sc = np.asarray(list(input_scalars) or [0.0], dtype=np.float64)
    _check(lib().mlkhip_execute_kernel(data, len(data), arch.encode(), sc.ctypes.data_as(_PD), len(input_scalars),
                                       out.ctypes.data_as(_PD), n_out))
    return [float(v) for v in out[:n_out]]


class DeviceBuffer:
    """Device memory owned from Python (through the library's HIP runtime)."""

    def __init__(self, elements: int, dtype: str):
        self.elements = int(elements)
        self.dtype = dtype
        self.code = DTYPE_CODE[dtype]
        self.nbytes = self.elements * np.dtype(NP_OF_CODE[self.code]).itemsize
        p = ctypes.c_void_p()
        _check(lib().mlkhip_malloc(ctypes.byref(p), max(self.nbytes, 16)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray, dtype: str) -> "DeviceBuffer":
        host = np.ascontiguousarray(np.asarray(a).astype(NP_OF_CODE[DTYPE_CODE[dtype]]).reshape(-1))
        buf = cls(host.size, dtype)
        if host.size:
            _check(lib().mlkhip_memcpy_h2d(buf.ptr, host.ctypes.data, buf.nbytes))
        return buf

    def fill_zero(self) -> None:
        _check(lib().mlkhip_fill32(self.ptr, 0, (self.nbytes + 3) // 4 * 4))

    def to_numpy(self) -> np.ndarray:
        out = np.empty(self.elements, dtype=NP_OF_CODE[self.code])
        if self.elements:
            _check(lib().mlkhip_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def binding(self) -> Binding:
        return Binding(self.ptr, self.elements, self.code, 0)

    def free(self) -> None:
        if self.ptr:
            lib().mlkhip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class LoadedKernel:
    """A built artifact (LoadedKernel analogue, backend_driver.h:110-183)."""

    def __init__(self, handle: int, km: KernelModule):
        self._h = ctypes.c_void_p(handle)
        self.module = km

    def __del__(self):
        try:
            if self._h:
                lib().mlkhip_release(self._h)
        except Exception:
            pass

    @property
    def class_name(self) -> str:
        return lib().mlkhip_class_name(self._h).decode()

    @property
    def policy(self) -> str:
        return lib().mlkhip_policy(self._h).decode()

    @property
    def is_multidim(self) -> bool:
        return bool(lib().mlkhip_is_multidim(self._h))

    def bindables(self) -> List[int]:
        return self.module.bindable_ids()

    @staticmethod
    def _scalars(scalars: Sequence[float]):
        sc = np.ascontiguousarray(np.asarray(list(scalars) or [0.0], dtype=np.float64))
        return sc, len(scalars)

    def run(self, arrays: Dict[int, np.ndarray], scalars: Sequence[float] = (), elements: int = 0,
            legacy: bool = False) -> Dict[int, np.ndarray]:
        """Host f64 artifact ABI (mlk_kernel multi-dim form, or the legacy 1-D
        form with ``legacy``). ``arrays`` maps buffer ids (inputs, and
        outputs to seed += / max stores) to arrays; every non-temp bindable
        gets an f64 array. Outputs come back by buffer id, and so does every
        input, as the call left it: a Store may target an input, and the
        reference then writes through the caller's array."""
        ids = self.bindables()
        host: List[Optional[np.ndarray]] = []
        for bid in ids:
            b = self.module.buffers[bid]
            if b.is_temp:
                host.append(None)
                continue
            n = _numel(b, elements)
            a = arrays.get(bid)
            h = np.zeros(n, dtype=np.float64) if a is None else \
                np.ascontiguousarray(np.asarray(a, dtype=np.float64).reshape(-1)).copy()
            host.append(h)
        ptrs = (_PD * max(1, len(ids)))(*[(h.ctypes.data_as(_PD) if h is not None else _PD())
                                          for h in host])
        sc, nsc = self._scalars(scalars)
        if legacy:
            rc = lib().mlkhip_kernel_1d(self._h, ptrs, len(ids), int(elements),
                                        sc.ctypes.data_as(_PD), nsc)
        else:
            dims = (ctypes.POINTER(ctypes.c_int64) * max(1, len(ids)))()
            rc = lib().mlkhip_kernel(self._h, ptrs, dims, len(ids), sc.ctypes.data_as(_PD), nsc,
                                     int(elements))
        _check(rc)
        return {bid: h for bid, h in zip(ids, host) if h is not None}

    def _bindings(self, bufs: Dict[int, DeviceBuffer]):
        ids = self.bindables()
        arr = (Binding * max(1, len(ids)))()
        for i, bid in enumerate(ids):
            b = self.module.buffers[bid]
            if bid in bufs:
                arr[i] = bufs[bid].binding()
            else:
                if not b.is_temp:
                    raise MlkHipError(BAD_BINDING, f"buffer {bid} ({b.name}) not bound")
                arr[i] = Binding(None, 0, DTYPE_CODE.get(b.dtype, F32), 0)
        return arr, len(ids)

    def run_device(self, bufs: Dict[int, DeviceBuffer], scalars: Sequence[float] = (),
                   elements: int = 0, stream: Optional[int] = None, sync: bool = True) -> None:
        arr, n = self._bindings(bufs)
        sc, nsc = self._scalars(scalars)
        _check(lib().mlkhip_run_device(self._h, arr, n, sc.ctypes.data_as(_PD), nsc,
                                       int(elements), stream))
        if sync:
            _check(lib().mlkhip_synchronize())

    def run_device_noalloc(self, bufs: Dict[int, DeviceBuffer], scalars: Sequence[float] = (),
                           elements: int = 0, stream: Optional[int] = None, sync: bool = True) -> None:
        """mlkhip_run_device_noalloc: scratch from the library's file-scope
        device array, nothing allocated."""
        arr, n = self._bindings(bufs)
        sc, nsc = self._scalars(scalars)
        _check(lib().mlkhip_run_device_noalloc(self._h, arr, n, sc.ctypes.data_as(_PD), nsc,
                                               int(elements), stream))
        if sync:
            _check(lib().mlkhip_synchronize())

    def time_device(self, bufs: Dict[int, DeviceBuffer], reps: int, warmup: int = 5,
                    scalars: Sequence[float] = (), elements: int = 0,
                    stream: Optional[int] = None) -> np.ndarray:
        arr, n = self._bindings(bufs)
        sc, nsc = self._scalars(scalars)
        ms = (ctypes.c_float * max(1, reps))()
        _check(lib().mlkhip_time_device(self._h, arr, n, sc.ctypes.data_as(_PD), nsc,
                                        int(elements), stream, warmup, reps, ms))
        return np.array(ms[:reps], dtype=np.float64)


    def time_device_span(self, bufs: Dict[int, DeviceBuffer], reps: int, warmup: int = 5,
                         scalars: Sequence[float] = (), elements: int = 0,
                         stream: Optional[int] = None) -> float:
        """Average ms per launch over `reps` back-to-back launches, one event
        pair around the span."""
        arr, n = self._bindings(bufs)
        sc, nsc = self._scalars(scalars)
        ms = ctypes.c_float(0.0)
        _check(lib().mlkhip_time_device_span(self._h, arr, n, sc.ctypes.data_as(_PD), nsc,
                                             int(elements), stream, warmup, reps, ctypes.byref(ms)))
        return float(ms.value)


    # ---- launch-form search (fastkernel analogue) ----
    def release_stream_scratch(self, stream=None) -> None:
        """Waits for `stream`, then frees the scratch set runs on it allocated."""
        _check(lib().mlkhip_release_stream_scratch(self._h, stream))

    def num_steps(self) -> int:
        return int(lib().mlkhip_num_steps(self._h))

    def step_variants(self, step: int) -> List[int]:
        out = (ctypes.c_int * 32)()
        n = lib().mlkhip_step_variants(self._h, step, out, 32)
        if n < 0:
            raise MlkHipError(BAD_BINDING, last_error())
        return list(out[:n])

    def step_kernel_name(self, step: int) -> str:
        """hipRTC kernel symbol of step `step` ("" for precompiled kernels)."""
        return lib().mlkhip_step_kernel_name(self._h, step).decode()

    def step_variant(self, step: int) -> int:
        return int(lib().mlkhip_step_variant(self._h, step))

    def set_step_variant(self, step: int, variant: int) -> None:
        _check(lib().mlkhip_set_step_variant(self._h, step, variant))

    @property
    def fingerprint(self) -> str:
        return lib().mlkhip_fingerprint(self._h).decode()

    @property
    def variants_from_cache(self) -> bool:
        return bool(lib().mlkhip_variants_from_cache(self._h))

    def autotune(self, bufs: Dict[int, DeviceBuffer], scalars: Sequence[float] = (), elements: int = 0,
                 reps: int = 10, cache_dir: Optional[str] = None) -> dict:
        """Certifies and times every launch form of every step on `bufs`
        (restored afterwards), keeps the fastest certified form per step and
        returns the search report."""
        arr, n = self._bindings(bufs)
        sc, nsc = self._scalars(scalars)
        cap = 1 << 16
        rep = ctypes.create_string_buffer(cap)
        _check(lib().mlkhip_autotune(self._h, arr, n, sc.ctypes.data_as(_PD), nsc, int(elements), int(reps),
                                     (cache_dir or "").encode(), rep, cap))
        return json.loads(rep.value.decode())


def _numel(b, elements: int) -> int:
    if b.dims:
        n = 1
        for d in b.dims:
            n *= int(d)
        return n
    return int(b.elements) if b.elements >= 0 else int(elements)


def build_hip_kernel_artifact(km: KernelModule,
                              config: Optional[HipBackendDriverConfig] = None,
                              reference_document: bool = False) -> LoadedKernel:
    """buildGpuKernelArtifact analogue (backend_driver.h:218-228). With
    ``reference_document`` the module crosses the boundary exactly as the
    reference's writer serializes it (KernelModule.to_reference_json)."""
    cfg = config or HipBackendDriverConfig()
    data = (km.to_reference_json() if reference_document else km.to_json()).encode()
    h = ctypes.c_void_p()
    rc = lib().mlkhip_build(data, len(data), cfg.arch.encode(),
                            (cfg.cache_dir or "").encode(), ctypes.byref(h))
    _check(rc)
    return LoadedKernel(h.value, km)


class HipBackend:
    """Convenience facade used by tests, smoke() and bench.py."""

    def __init__(self, arch: str = "gfx950"):
        self.arch = arch
        lib()

    def device_available(self) -> bool:
        return bool(lib().mlkhip_device_available(self.arch.encode()))

    def build(self, km: KernelModule, cache_dir: Optional[str] = None,
              reference_document: bool = False) -> LoadedKernel:
        return build_hip_kernel_artifact(km, HipBackendDriverConfig(self.arch, cache_dir), reference_document)
