"""Writes tests/golden/oracle_golden.json: small vectors from the CPU oracle
(oracle/oracle.cpp) for each hot-path config at reduced shapes, the reference's
own known answers, and the first SplitMix64 outputs.

The reference cannot run here (its translation units need <expected>), so the
vectors are the oracle's, which tests/test_oracle.py pins against the
reference's fixtures and its poly7 header. They guard the oracle and the input
generator against drift: tests/test_golden.py recomputes every vector and
requires bit-identical results.

    python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from mlk2_amd import fixtures as fx  # noqa: E402
from mlk2_amd import inputs  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_golden.json")


def splitmix_reference(seed, n):
    """Pure-Python SplitMix64 counter mode (independent of inputs.py's numpy form)."""
    out = []
    mask = (1 << 64) - 1
    for i in range(n):
        z = (seed + i * 0x9E3779B97F4A7C15) & mask
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        out.append(z ^ (z >> 31))
    return out


def summary(a):
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float64).reshape(-1))
    return {
        "n": int(a.size),
        "head": [float(v).hex() for v in a[:16]],
        "tail": [float(v).hex() for v in a[-16:]],
        "sha256": hashlib.sha256(a.tobytes()).hexdigest(),
    }


def cases():
    """(name, module builder, input builder, output buffer id)."""
    return [
        ("c1_n4096", lambda: fx.config1_module(n=4096),
         lambda: {0: inputs.config_inputs("c1", {"n": 4096})["x"]}, 1),
        ("c2_64x4096_call", lambda: fx.config2_module(64, 4096, 1),
         lambda: {0: inputs.config_inputs("c2", {"m": 64, "k": 4096})["x"]}, 1),
        ("c2_16x512_nest", lambda: fx.config2_module(16, 512, 2),
         lambda: {0: inputs.config_inputs("c2", {"m": 16, "k": 512})["x"]}, 1),
        ("c3_64x256_nest", lambda: fx.config3_module(64, 256, 2),
         lambda: dict(zip((0, 1), inputs.config_inputs("c3", {"rows": 64, "cols": 256}).values())), 2),
        ("c4a_64x64x64_nest", lambda: fx.config4_module(64, 64, 64, "f32", 2),
         lambda: dict(zip((0, 1), inputs.config_inputs("c4a", {"m": 64, "k": 64, "n": 64}).values())), 2),
        ("c4b_128x256x64_call", lambda: fx.config4_module(128, 256, 64, "f16", 1),
         lambda: dict(zip((0, 1), inputs.config_inputs("c4b", {"m": 128, "k": 256, "n": 64}).values())), 2),
        ("c5_2x32x16", lambda: fx.score_softmax_module(2, 32, 16),
         lambda: dict(zip((0, 1, 2), inputs.config_inputs("c5", {"batch": 2, "seq": 32, "dim": 16}).values())), 3),
    ]


def build():
    doc = {"generator": "SplitMix64 counter mode, see mlk2_amd/inputs.py",
           "splitmix64_seed_0x5EED0001_first8": [hex(v) for v in splitmix_reference(0x5EED0001, 8)],
           "known_answers": {
               # examples/scalar/README.md:9, tests/differential/differential_test.cpp:44-48
               "sin_graph_at_2": {"x": 2.0, "y": -0.5440211108893698, "tol": 1e-13},
           },
           "cases": {}}
    # Reference GEMM fixture (tests/unit/unit_poly.cpp:2024-2056): exact outputs.
    M, K, N = 8, 6, 7
    A = np.array([((i * 7) % 13) * 0.25 for i in range(M * K)])
    B = np.array([((i * 5) % 11) * 0.5 for i in range(K * N)])
    C = oracle.run(fx.matmul_call_module(M, K, N, "f64", "f64"), {0: A, 1: B})[2]
    doc["known_answers"]["gemm_8x6x7_unit_poly"] = {"C": [float(v).hex() for v in C]}
    for name, mk, mkin, out_id in cases():
        km = mk()
        ins = mkin()
        out = oracle.run(km, ins, hw_threads=1)[out_id]
        doc["cases"][name] = {"output_buffer": out_id, **summary(out)}
    return doc


if __name__ == "__main__":
    doc = build()
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {OUT}: {len(doc['cases'])} cases")
