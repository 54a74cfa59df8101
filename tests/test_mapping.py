"""Index mapping of the hand-written kernels at the full configuration shapes,
bit for bit.

Each input encodes where it sits (its flat index, a permutation, a set of
columns per row) and the operations are exact on those values, so every
output element has exactly one correct value: the one the walker computes at
that element's flat address. A kernel that skips an instance, writes one
twice with different values, or reads or writes the wrong address fails the
equality. This is the tile-schedule mapping check of the reference's CUDA
geometry tests (backends/cpu/tests/unit_poly.cpp:4810-4922) restated as
end-to-end data; every launch form a kernel declares is run.

The *_expected_values_match_oracle tests pin each expected-value rule on
the CPU oracle at a reduced shape.
"""
import sys

import numpy as np
import pytest

import oracle
from mlk2_amd import fixtures as fx
from mlk2_amd.backend import DeviceBuffer
from mlk2_amd.kernel_ir import KernelExpr, const, elem_a, scalar


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _forms(art):
    return art.step_variants(0) or [-1]


def _column_hash(n, seed):
    j = np.arange(n, dtype=np.uint64)
    h = (j * np.uint64(0x9E3779B97F4A7C15) + np.uint64(seed)) >> np.uint64(33)
    return (h & np.uint64(0xFF)).astype(np.int64)


@pytest.mark.gpu
def test_c1_shape_identity_chain(hip):
    # The elementwise-1d template at C1's 2^24 elements: y = x * 1 with
    # x[i] = i (exact in f32 below 2^24).
    n = 1 << 24
    say(f"mapping c1-shape identity n={n}")
    km = fx.lower_elementwise([("x", [n], "f32")], [KernelExpr("mul", elem_a(), const(1.0))], [n], "f32")
    art = hip.build(km)
    assert art.class_name == "elementwise-1d"
    x = np.arange(n, dtype=np.float32)
    bufs = {0: DeviceBuffer.from_array(x, "f32"), 1: DeviceBuffer(n, "f32")}
    bufs[1].fill_zero()
    art.run_device(bufs)
    assert np.array_equal(bufs[1].to_numpy(), x)


def _c3_case(rows, cols):
    # y = exp(0 * x + b[j]) * x with x the flat index and b[j] in {0, -inf}:
    # y is x where b[j] == 0 and exactly 0 where b[j] == -inf.
    x = np.arange(rows * cols, dtype=np.float32)
    b = np.where(_column_hash(cols, 3) % 3 == 1, -np.inf, 0.0).astype(np.float32)
    want = np.where(np.tile(b, rows) == 0.0, x, np.float32(0.0))
    return x, b, want


def test_c3_expected_values_match_oracle():
    # Pins the expected-value rule (exp(-inf) = 0, 0 * x = 0) on the oracle
    # at a reduced shape.
    rows, cols = 16, 64
    x, b, want = _c3_case(rows, cols)
    km = fx.config3_module(rows, cols, 2, a_operand=scalar(0))
    got = oracle.run(km, {0: x, 1: b}, scalars=[0.0])[2]
    assert np.array_equal(got.astype(np.float32), want)


@pytest.mark.gpu
def test_c3_full_shape_broadcast_mapping(hip):
    rows = cols = 4096
    say("mapping c3 4096x4096")
    x, b, want = _c3_case(rows, cols)
    km = fx.config3_module(rows, cols, 2, a_operand=scalar(0))
    art = hip.build(km)
    assert art.class_name == "elementwise-nd"
    bufs = {0: DeviceBuffer.from_array(x, "f32"), 1: DeviceBuffer.from_array(b, "f32"),
            2: DeviceBuffer(rows * cols, "f32")}
    bufs[2].fill_zero()
    art.run_device(bufs, scalars=[0.0])
    assert np.array_equal(bufs[2].to_numpy(), want)


def _softmax_rows(rows, cols, hot=4):
    # `hot` distinct columns per row hold 0, every other entry -inf: each
    # row's softmax is exactly 1/hot at those columns and 0 elsewhere.
    rng = np.random.default_rng(11)
    x = np.full((rows, cols), -np.inf, dtype=np.float32)
    want = np.zeros((rows, cols), dtype=np.float32)
    r = np.arange(rows)[:, None]
    picks = np.argsort(rng.random((rows, cols)), axis=1)[:, :hot] if cols <= 512 else \
        np.stack([rng.choice(cols, hot, replace=False) for _ in range(rows)])
    x[r, picks] = 0.0
    want[r, picks] = np.float32(1.0 / hot)
    return x, want


def test_softmax_expected_values_match_oracle():
    x, want = _softmax_rows(12, 64)
    got = oracle.run(fx.config2_module(12, 64, 2), {0: x})[1]
    assert np.array_equal(got.astype(np.float32).reshape(12, 64), want)


@pytest.mark.gpu
def test_c2_full_shape_row_mapping_every_form(hip):
    rows, cols = 8192, 4096
    x, want = _softmax_rows(rows, cols)
    art = hip.build(fx.config2_module(rows, cols, 2))
    bufs = {0: DeviceBuffer.from_array(x, "f32"), 1: DeviceBuffer(rows * cols, "f32")}
    for v in _forms(art):
        say(f"mapping c2 8192x4096 form {v}")
        art.set_step_variant(0, v)
        bufs[1].fill_zero()
        art.run_device(bufs)
        assert np.array_equal(bufs[1].to_numpy().reshape(rows, cols), want), v


def _perm_gemm(m, k, n, dtype):
    # A = a row permutation (A[i, p(i)] = 1), B encodes (k, n): C = B[p, :]
    # exactly (one nonzero product per sum). With m > k the indices wrap
    # modulo k: rows that share a source row are interchangeable, but a
    # misplaced tile of 64 or 256 rows still shows.
    rng = np.random.default_rng(5)
    p = (rng.permutation(max(m, k)) % k)[:m]
    A = np.zeros((m, k), dtype=np.float32)
    A[np.arange(m), p] = 1.0
    kk, nn = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    if dtype == "f32":
        B = (kk * n + nn).astype(np.float32)            # < 2^24: exact
    else:
        B = (((kk * 37 + nn * 11) % 2039) - 1019).astype(np.float32)   # exact in f16
    return A, B, B[p, :]


def test_gemm_expected_values_match_oracle():
    A, B, want = _perm_gemm(8, 12, 7, "f16")
    got = oracle.run(fx.config4_module(8, 12, 7, "f16", 2), {0: A, 1: B})[2]
    assert np.array_equal(got.astype(np.float32).reshape(8, 7), want)


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n,dtype", [(1024, 1024, 1024, "f32"), (4096, 4096, 4096, "f16"),
                                         # non-square grids: f32 tiles of 64, f16 tiles of 256
                                         # row-major (3 x 5) and in XCD groups of 4 x 8
                                         # (8 x 32 and 32 x 8 tiles)
                                         (192, 256, 320, "f32"), (2048, 128, 512, "f32"),
                                         (512, 128, 2048, "f32"),
                                         (768, 1024, 1280, "f16"), (2048, 2048, 8192, "f16"),
                                         (8192, 256, 2048, "f16")])
def test_gemm_full_shape_mapping_every_form(hip, m, k, n, dtype):
    A, B, want = _perm_gemm(m, k, n, dtype)
    art = hip.build(fx.config4_module(m, k, n, dtype, 2))
    assert art.class_name == "gemm-nest"
    bufs = {0: DeviceBuffer.from_array(A, dtype), 1: DeviceBuffer.from_array(B, dtype),
            2: DeviceBuffer(m * n, "f32")}
    for v in _forms(art):
        say(f"mapping gemm {dtype} {m}x{k}x{n} form {v}")
        art.set_step_variant(0, v)
        bufs[2].fill_zero()
        art.run_device(bufs)
        assert np.array_equal(bufs[2].to_numpy().reshape(m, n), want), v


def _score_case(batch, seq, dim):
    # Q[b,i] and K[b,j] are 64 * unit vectors on axis (i + 5b) % dim and
    # (j + 5b) % dim: the score is 4096/sqrt(dim) where i = j (mod dim) and 0
    # elsewhere. exp of (0 - max) underflows to 0 in f32, so each row is
    # exactly 1/(seq/dim) on its seq/dim matching columns and 0 elsewhere.
    Q = np.zeros((batch, seq, dim), dtype=np.float32)
    K = np.zeros((batch, seq, dim), dtype=np.float32)
    i = np.arange(seq)
    for b in range(batch):
        Q[b, i, (i + 5 * b) % dim] = 64.0
        K[b, i, (i + 5 * b) % dim] = 64.0
    bias = np.zeros(seq, dtype=np.float32)
    hit = (i[:, None] % dim) == (i[None, :] % dim)
    row = np.where(hit, np.float32(dim / seq), np.float32(0.0)).astype(np.float32)
    want = np.broadcast_to(row, (batch, seq, seq)).reshape(batch * seq, seq)
    return Q, K, bias, want


def test_score_expected_values_match_oracle():
    Q, K, bias, want = _score_case(2, 64, 16)
    got = oracle.run(fx.score_softmax_module(2, 64, 16), {0: Q, 1: K, 2: bias})[3]
    assert np.array_equal(got.astype(np.float32).reshape(128, 64), want)


@pytest.mark.gpu
def test_c5_full_shape_mapping_every_form(hip):
    batch, seq, dim = 16, 2048, 128
    Q, K, bias, want = _score_case(batch, seq, dim)
    art = hip.build(fx.score_softmax_module(batch, seq, dim))
    assert art.class_name == "score-softmax"
    bufs = {0: DeviceBuffer.from_array(Q, "f16"), 1: DeviceBuffer.from_array(K, "f16"),
            2: DeviceBuffer.from_array(bias, "f32"), 3: DeviceBuffer(batch * seq * seq, "f32")}
    for v in _forms(art):
        say(f"mapping c5 16x2048x128 form {v}")
        art.set_step_variant(0, v)
        bufs[3].fill_zero()
        art.run_device(bufs)
        got = bufs[3].to_numpy().reshape(batch * seq, seq)
        assert np.array_equal(got, want), v
