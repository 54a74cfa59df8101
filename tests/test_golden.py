"""Golden vectors (tests/golden/oracle_golden.json, made by make_golden.py):
the oracle and the input generator must reproduce them bit-for-bit."""
import json
import os

import numpy as np
import pytest

import oracle
from mlk2_amd import fixtures as fx
from mlk2_amd import inputs

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "oracle_golden.json")))

import importlib.util
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


def test_splitmix_numpy_matches_pure_python():
    want = [int(v, 16) for v in GOLDEN["splitmix64_seed_0x5EED0001_first8"]]
    got = [int(v) for v in inputs.splitmix64(0x5EED0001, 8)]
    assert got == want == make_golden.splitmix_reference(0x5EED0001, 8)
    u = inputs.unit(0x5EED0001, 8)
    assert np.array_equal(u, np.array([(v >> 40) * 2.0 ** -24 for v in want]))


def test_known_answer_sin_graph():
    ka = GOLDEN["known_answers"]["sin_graph_at_2"]
    y = oracle.run(fx.config1_module(n=1, dtype="f64"), {0: np.array([ka["x"]])})[1][0]
    assert abs(y - ka["y"]) <= ka["tol"]


def test_reference_gemm_fixture():
    M, K, N = 8, 6, 7
    A = np.array([((i * 7) % 13) * 0.25 for i in range(M * K)])
    B = np.array([((i * 5) % 11) * 0.5 for i in range(K * N)])
    C = oracle.run(fx.matmul_call_module(M, K, N, "f64", "f64"), {0: A, 1: B})[2]
    assert [float(v).hex() for v in C] == GOLDEN["known_answers"]["gemm_8x6x7_unit_poly"]["C"]


@pytest.mark.parametrize("case", [c[0] for c in make_golden.cases()])
def test_oracle_reproduces_golden(case):
    name, mk, mkin, out_id = next(c for c in make_golden.cases() if c[0] == case)
    out = oracle.run(mk(), mkin(), hw_threads=1)[out_id]
    assert make_golden.summary(out) == {k: v for k, v in GOLDEN["cases"][case].items()
                                        if k != "output_buffer"}

