"""The work model and the parity gates, on the CPU.

* Essential work and the roofline lower bound: the reference's own cases
  (tests/unit/unit_fastkernel.cpp:221-264) through mlkhip_essential_work,
  plus the element sizes this backend prices by dtype.
* The gates of tools/mlk-poly/poly_bench.cpp (ULP distance :78-93, the
  Rule-43 bit-exact gate :211-224, the policy-driven GPU gate :499-575),
  pinned on values whose distances are known by construction.
"""
import numpy as np

from mlk2_amd import backend as be
from mlk2_amd import fixtures as fx
from mlk2_amd.kernel_ir import KernelExpr, const, elem_a
from mlk2_amd.parity import bit_exact, max_rel, policy_gate, ulp_distance_f32, ulp_distance_f64


# ---- work model (fastkernel essentialWorkModel / rooflineLowerBound) ----
def test_essential_work_reference_gemm_case():
    # tests/unit/unit_fastkernel.cpp:221-236: GEMM 4x3x2 over f64 buffers:
    # O_min = 2*4*3*2 = 48, B_min = 8 * (12 + 6 + 8) = 208, and with 1000 B/s
    # and 100 op/s the lower bound is max(0.208, 0.48) = 0.48 s.
    w = be.essential_work(fx.matmul_call_module(4, 3, 2, "f64", "f64"), 1000.0, 100.0)
    assert (w["min_ops"], w["min_bytes"], w["ops_known"], w["bytes_known"]) == (48, 208, True, True)
    assert abs(w["roofline_lower_sec"] - 0.48) < 1e-12


def test_essential_work_unknown_extent_gives_no_bound():
    # unit_fastkernel.cpp:238-264: a dynamic extent without dims leaves the
    # bytes unknown, and then there is no bound.
    km = fx.lower_elementwise([("x", [8], "f32")], [KernelExpr("mul", elem_a(), const(2.0))], [8], "f32")
    km.buffers[0].elements = -1
    km.buffers[0].dims = []
    km.buffers[1].elements = -1
    km.buffers[1].dims = []
    km.nodes[2].end = -1
    w = be.essential_work(km, 1000.0, 100.0)
    assert not w["bytes_known"] and w["roofline_lower_sec"] == 0.0


def test_essential_work_dtype_sizes_and_walk():
    # Element sizes follow the buffers' dtypes (the reference prices every
    # element at 8 B). The walk starts from every node and recurses, so the
    # 4-expression chain nested in its loop counts twice, as in the reference.
    w = be.essential_work(fx.config1_module(1024), 8e12, 157.3e12)
    assert (w["min_bytes"], w["min_ops"]) == (1024 * 4 * 2, 8)
    w = be.essential_work(fx.config4_module(64, 64, 64, "f16", 1))
    assert (w["min_bytes"], w["min_ops"]) == (64 * 64 * 2 * 2 + 64 * 64 * 4, 2 * 64 ** 3)
    assert abs(w["roofline_lower_sec"] - max(w["min_bytes"] / 8e12, w["min_ops"] / 2.5e15)) < 1e-18
    w = be.essential_work(fx.softmax_call_module(8, 16))
    assert w["min_ops"] == 5 * 8 * 16


# ---- gates (poly_bench.cpp:78-93, :211-224, :499-575) -------------------
def test_ulp_distance_f64_known_values():
    one = np.array([1.0])
    assert ulp_distance_f64(one, np.nextafter(one, 2.0))[0] == 1.0
    assert ulp_distance_f64(np.array([-0.0]), np.array([0.0]))[0] == 0.0
    tiny = np.array([5e-324])
    assert ulp_distance_f64(-tiny, tiny)[0] == 2.0            # across zero
    assert ulp_distance_f64(np.array([np.nan]), np.array([np.nan]))[0] == 0.0
    assert ulp_distance_f64(np.array([np.nan]), one)[0] == np.inf
    m = np.array([-1.0])
    assert ulp_distance_f64(m, np.nextafter(m, -2.0))[0] == 1.0


def test_ulp_distance_f32_known_values():
    one = np.array([1.0], dtype=np.float32)
    assert ulp_distance_f32(np.nextafter(one, np.float32(2.0)), np.array([1.0]))[0] == 1.0
    assert ulp_distance_f32(np.array([0.0], dtype=np.float32), np.array([-0.0]))[0] == 0.0
    assert ulp_distance_f32(np.array([np.nan], dtype=np.float32), np.array([1.0]))[0] == np.inf


def test_bit_exact_nan_never_matches():
    assert bit_exact(np.array([1.0, -0.0]), np.array([1.0, 0.0])) == (True, -1)
    assert bit_exact(np.array([1.0, np.nan]), np.array([1.0, np.nan])) == (False, 1)
    assert bit_exact(np.array([1.0, 2.0]), np.array([1.0, np.nextafter(2.0, 3.0)])) == (False, 1)


def test_max_rel_special_values():
    # math_bench.cpp:172-181: |got - ref| / max(|ref|, 1), where a NaN error
    # (inf - inf, or a NaN operand) never raises the maximum.
    inf, nan = np.inf, np.nan
    assert max_rel(np.array([3.0, -0.5]), np.array([2.0, -0.25])) == 0.5     # 1/2 and 0.25/1
    assert max_rel(np.array([inf, -inf, 1.0]), np.array([inf, -inf, 1.0])) == 0.0   # equal infinities
    assert max_rel(np.array([nan, 1.0]), np.array([nan, 1.0])) == 0.0
    assert max_rel(np.array([inf]), np.array([-inf])) == inf
    assert max_rel(np.array([inf]), np.array([1e300])) == inf
    # Stricter than the reference: a NaN on one side only fails.
    assert max_rel(np.array([nan]), np.array([1.0])) == inf
    assert max_rel(np.array([1.0]), np.array([nan])) == inf


def test_policy_gates():
    ref = np.array([1.0, 2.0, -3.0])
    assert policy_gate("bitexact-rne-gfx950-v1", ref.copy(), ref)[0]
    f = ref.astype(np.float32)
    bumped = f.copy()
    bumped[1] = np.nextafter(np.nextafter(bumped[1], np.float32(9)), np.float32(9))
    ok, d, _ = policy_gate("tol-4ulp-f32-gfx950-v1", bumped, ref)
    assert ok and d == 2.0
    ok, e, _ = policy_gate("tol-rel1e-6-gfx950-v1", ref + 2e-6, ref)
    assert not ok and abs(e - 2e-6) < 1e-12
    assert policy_gate("tol-rel1e-5sqrtk-gfx950-v1", ref + 2e-5, ref, k=16)[0]      # 4e-5 allowed
    assert not policy_gate("tol-rel1e-5sqrtk-gfx950-v1", ref + 2e-5, ref, k=1)[0]
    assert policy_gate("tol-rel1e-2-gfx950-v1", ref * 1.005, ref)[0]
