"""Generated text is a pure function of the module.

The reference pins that its emitted device source is the same text every time
it is emitted for one module (tests/unit/unit_poly.cpp:4169-4183). Here two
kinds of generated text feed cache keys and fingerprints: the hipRTC instance
source of each elementwise and loop-nest step (its hash names the kernel
symbol and keys the instance cache), and the per-module artifact source that
mlkhip_emit_artifact writes (host/artifact.cpp). Each is emitted twice in one
process, and again after the execute-route cache is cleared, and compared
byte for byte. No device needed.
"""
import ctypes
import os

import pytest

import nest_fuzz as nf
from mlk2_amd import backend as be
from mlk2_amd import fixtures as fx
from test_artifact import emit
from test_host import EXP_CASES


def source_modules():
    return [
        ("c1", fx.config1_module(n=1 << 14)),
        ("c1-lifted", fx.lift_1d(fx.config1_module(n=1 << 14))),
        ("c2-synth-reader", fx.softmax_rowmax_reader_module(64, 512)),
        ("c3", fx.config3_module(64, 512, tier=2)),
        ("exp*b", fx.lower_elementwise([("a", [4096], "f32"), ("b", [4096], "f32")], EXP_CASES[0][1], [4096])),
        ("fuzz-3", nf.random_module(3)),
        ("fuzz-11", nf.random_module(11, exact_ops=False)),
        ("fuzz-tiled-5", nf.tiled_random_module(5)),
    ]


def step_sources(km):
    n = be.plan(km)[2]
    out = []
    for s in range(n):
        size, src = be.compile_check(km, s)
        out.append((size, src))
    return out


@pytest.mark.parametrize("label,km", source_modules(), ids=[m[0] for m in source_modules()])
def test_instance_source_is_reemitted_byte_for_byte(label, km):
    first = step_sources(km)
    assert any(src for _, src in first), label       # at least one hipRTC step
    second = step_sources(km)
    be.lib().mlkhip_execute_cache_clear()
    third = step_sources(km)
    for (n1, s1), (n2, s2), (n3, s3) in zip(first, second, third):
        assert s1 == s2 == s3
        assert n1 == n2 == n3                       # the same code-object size
    # The module as the reference's writer serializes it (kernel_ir.cpp:
    # 97-254: "math" on Compute nodes only, NaN as null, +-inf clamped)
    # gives the same text.
    text = km.to_reference_json().encode()
    for s, (_, src) in enumerate(first):
        buf = ctypes.create_string_buffer(1 << 20)
        assert be.lib().mlkhip_compile_check(text, len(text), s, b"gfx950", buf, 1 << 20) >= 0
        assert buf.value.decode() == src


def artifact_modules():
    return [
        ("c1", fx.config1_module(n=1 << 14)),
        ("c2", fx.config2_module(64, 512, tier=2)),
        ("c3", fx.config3_module(64, 512, tier=2)),
        ("c4a-call", fx.config4_module(256, 128, 256, "f32", tier=1)),
        ("c4b", fx.config4_module(256, 256, 256, "f16", tier=2)),
        ("c5", fx.score_softmax_module(2, 256, 128)),
    ]


@pytest.mark.parametrize("label,km", artifact_modules(), ids=[m[0] for m in artifact_modules()])
def test_artifact_source_is_reemitted_byte_for_byte(tmp_path, label, km):
    texts = []
    for i in range(3):
        d = tmp_path / f"emit{i}"
        d.mkdir()
        if i == 2:
            be.lib().mlkhip_execute_cache_clear()
        emit(km, d)
        texts.append(open(os.path.join(d, "mlk_kernel.cpp"), "rb").read())
    assert texts[0] == texts[1] == texts[2]
