"""Parity gates: the comparisons the reference's bench and tests apply.

* ``ulp_distance_f64`` restates ``tools/mlk-poly/poly_bench.cpp:78-93``
  (ordered-bit distance; NaN pairs equal, one-sided NaN infinite, +/-0 equal).
* ``ulp_distance_f32`` is the same over f32 bit patterns: the GPU value
  against the f64 reference rounded to f32.
* ``max_rel`` restates ``bench/math/math_bench.cpp:172-181``:
  ``|got - ref| / max(|ref|, 1)``. There a NaN error never raises the
  maximum, so equal infinities (inf - inf) count as no error; they do here
  too. A NaN on one side only is also skipped there; here it counts as an
  infinite error, so a gate cannot pass over a NaN the reference does not
  produce.
* ``bit_exact`` restates the Rule-43 element gate
  (``tools/mlk-poly/poly_bench.cpp:211-224``): no element differs under
  ``!=``, so a NaN never matches, not even a NaN.
* ``policy_gate`` is the policy-driven gate of the GPU rows
  (``poly_bench.cpp:499-575``) for this backend's policy ids: bit-exact
  policies gate with ``bit_exact``, the others with their tolerance on the
  measured ULP distance or relative error.
"""
from __future__ import annotations

import numpy as np


def ulp_distance_f32(got: np.ndarray, ref_f64: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(got, dtype=np.float32).reshape(-1)
    r = np.ascontiguousarray(np.asarray(ref_f64, dtype=np.float64).astype(np.float32)).reshape(-1)
    gb = g.view(np.uint32).astype(np.int64)
    rb = r.view(np.uint32).astype(np.int64)
    go = np.where(gb >= (1 << 31), (1 << 31) - gb, gb)
    ro = np.where(rb >= (1 << 31), (1 << 31) - rb, rb)
    d = np.abs(go - ro).astype(np.float64)
    gn, rn = np.isnan(g), np.isnan(r)
    d = np.where(gn & rn, 0.0, d)
    d = np.where(gn ^ rn, np.inf, d)
    d = np.where(g == r, 0.0, d)
    return d


def ulp_distance_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float64).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.float64).reshape(-1)
    ab = a.view(np.int64)
    bb = b.view(np.int64)
    lo = np.int64(-0x7FFFFFFFFFFFFFFF - 1)
    with np.errstate(over="ignore"):
        ao = np.where(ab >= 0, ab, lo - ab)
        bo = np.where(bb >= 0, bb, lo - bb)
        d = np.abs((ao - bo).astype(np.float64))
    an, bn = np.isnan(a), np.isnan(b)
    d = np.where(an & bn, 0.0, d)
    d = np.where(an ^ bn, np.inf, d)
    d = np.where(a == b, 0.0, d)
    return d


def max_rel(got: np.ndarray, ref: np.ndarray) -> float:
    g = np.asarray(got, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    if g.size == 0:
        return 0.0
    denom = np.maximum(np.abs(r), 1.0)
    with np.errstate(invalid="ignore"):
        e = np.abs(g - r) / denom
    both_nan = np.isnan(g) & np.isnan(r)
    e = np.where(both_nan | (g == r), 0.0, e)
    e = np.where(np.isnan(e), np.inf, e)
    return float(e.max())


def bit_exact(got: np.ndarray, ref: np.ndarray):
    """(passed, first differing index or -1): every element equal under !=
    semantics, so NaN anywhere fails."""
    g = np.asarray(got, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    if g.shape != r.shape:
        return False, 0
    diff = np.nonzero(~(g == r))[0]
    return (diff.size == 0), (int(diff[0]) if diff.size else -1)


def policy_gate(policy: str, got: np.ndarray, ref: np.ndarray, k: int = 1):
    """(passed, measure, note) of an artifact's output under its tolerance
    policy id (``mlkhip_policy``): the measure is the first differing index
    for bit-exact policies, the max f32 ULP distance for the 4-ULP policy,
    and the max relative error for the relative ones."""
    if policy.startswith("bitexact"):
        ok, idx = bit_exact(got, ref)
        return ok, float(idx), "bit-exact-policy"
    if policy.startswith("tol-4ulp"):
        d = float(ulp_distance_f32(got, ref).max()) if np.size(ref) else 0.0
        return d <= 4.0, d, f"ulp-bounded-policy max={d:g} ulp (measured)"
    if policy.startswith("tol-rel1e-5sqrtk"):
        tol = 1e-5 * float(np.sqrt(k))
    elif policy.startswith("tol-rel1e-6"):
        tol = 1e-6
    elif policy.startswith("tol-rel1e-2"):
        tol = 1e-2
    else:
        raise ValueError(f"unknown policy {policy!r}")
    e = max_rel(got, ref)
    return e <= tol, e, f"relative-policy max={e:.3g} (tolerance {tol:g})"
