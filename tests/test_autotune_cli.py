"""`python -m mlk2_amd.autotune`: the reference's `mlk-poly autotune` verb
(tools/mlk-poly/mlk_poly.cpp:389-600) extended from its f64 GEMM to the five
configs. CPU tests cover the command line and the modules it builds; the
GPU test runs the search and reads its report."""
import json
import sys

import numpy as np
import pytest

from mlk2_amd import autotune as at


def test_defaults_are_the_reference_gemm():
    a = at.parse_args([])
    assert a.configs == ["gemm"] and a.dtype == "f64" and a.reps == 10
    title, km, arrays = at.config_case("gemm", a)
    # mlk_poly.cpp:392: m = 64, k = 48, n = 56, f64.
    assert title.startswith("gemm f64 64x48x56")
    assert [x.shape for x in arrays] == [(64, 48), (48, 56)]
    assert [b.dtype for b in km.buffers if b.is_input] == ["f64", "f64"]


def test_all_selects_every_config():
    assert at.parse_args(["--config=all"]).configs == list(at.CONFIGS)


@pytest.mark.parametrize("argv", [["--config=c9"], ["--dtype=f8"], ["--tier=3"], ["--reps=0"], ["--m=0"],
                                  ["--bogus=1"]])
def test_usage_errors(argv):
    with pytest.raises(at.UsageError):
        at.parse_args(argv)
    assert at.main(argv) == 2


@pytest.mark.parametrize("name,argv,shapes", [
    ("c1", ["--elements=4096"], [(4096,)]),
    ("c2", ["--rows=64", "--cols=256"], [(64, 256)]),
    ("c3", ["--rows=32", "--cols=64"], [(32, 64), (64,)]),
    ("c4a", ["--m=64", "--k=64", "--n=64"], [(64, 64), (64, 64)]),
    ("c4b", ["--m=256", "--k=64", "--n=256"], [(256, 64), (64, 256)]),
    ("c5", ["--batch=1", "--seq=256", "--dim=128"], [(1, 256, 128), (1, 256, 128), (256,)]),
])
def test_config_cases_follow_the_shapes(name, argv, shapes):
    a = at.parse_args([f"--config={name}"] + argv)
    title, km, arrays = at.config_case(name, a)
    assert title.startswith(name)
    assert [np.asarray(x).shape for x in arrays] == shapes
    ins = [b for b in km.buffers if b.is_input]
    assert len(ins) == len(arrays)
    for b, x in zip(ins, arrays):
        assert b.elements == np.asarray(x).size


def test_no_device_is_a_usage_exit(monkeypatch):
    monkeypatch.setattr(at.be.HipBackend, "device_available", lambda self: False)
    assert at.main(["--config=c1", "--elements=1024"]) == 2


@pytest.mark.gpu
def test_search_over_configs_writes_its_report(tmp_path, capsys):
    out = tmp_path / "report.json"
    rc = at.main(["--config=gemm,c1,c4a,c4b,c5", "--m=256", "--k=128", "--n=256", "--elements=65536",
                  "--batch=1", "--seq=512", "--dim=128", "--reps=3", f"--cache-dir={tmp_path}",
                  f"--json-out={out}"])
    text = capsys.readouterr().out
    print(text, flush=True)
    sys.stdout.flush()
    assert rc == 0
    rep = json.loads(out.read_text())
    assert set(rep) == {"gemm", "c1", "c4a", "c4b", "c5"}
    # One form only: the search times nothing.
    assert rep["gemm"]["steps"] == [] and rep["c1"]["steps"] == []
    # Searched steps: every declared form is a candidate and the chosen one
    # is certified.
    for name, forms in (("c4a", [0, 1]), ("c4b", [8, 7, 0, 1, 2, 3, 5, 6]), ("c5", [0, 1])):
        (st,) = rep[name]["steps"]
        assert [c["variant"] for c in st["candidates"]] == forms, name
        chosen = [c for c in st["candidates"] if c["variant"] == st["chosen"]][0]
        assert chosen["admissible"] and chosen["certificate"]["identity"]["certified"], name
        assert rep[name]["combined_certified"] is True
        assert rep[name]["cache"]["file"].startswith(str(tmp_path))
    # The launch certificate counts the tiles of the form that runs: 64 x 64
    # for f32, 256 x 256 for f16 (128 x 256 under forms 5 and 6).
    assert rep["c4a"]["steps"][0]["launch"]["workgroups"] == 16
    assert rep["c4b"]["steps"][0]["launch"]["workgroups"] in (1, 2)
    assert "== fast-kernel search: c4b gemm f16 256x128x256" in text
    assert "<- chosen" in text


def test_module_document_case(tmp_path):
    # --module takes an mlk-kernel document as written; inputs are seeded
    # and sized from its buffer table.
    from test_nest import generic, weighted_rows_module
    km = generic(weighted_rows_module())
    doc = tmp_path / "nest.json"
    doc.write_text(km.to_json())
    a = at.parse_args([f"--module={doc}"])
    assert a.configs == ["module"]
    title, mod, arrays = at.config_case("module", a)
    assert mod.to_json() == km.to_json()
    assert mod.bindable_ids() == km.bindable_ids()
    ins = [i for i, b in enumerate(km.buffers) if b.is_input and not b.is_temp]
    assert [x.size for x in arrays] == [km.buffers[i].elements for i in ins]
    bad = tmp_path / "bad.json"
    bad.write_text('{"format": "other"}')
    with pytest.raises(at.UsageError):
        at.config_case("module", at.parse_args([f"--module={bad}"]))


@pytest.mark.gpu
def test_module_document_search(tmp_path, capsys):
    from test_nest import generic, weighted_rows_module
    km = generic(weighted_rows_module())
    doc = tmp_path / "nest.json"
    doc.write_text(km.to_json())
    out = tmp_path / "report.json"
    rc = at.main([f"--module={doc}", "--reps=3", f"--cache-dir={tmp_path}", f"--json-out={out}"])
    print(capsys.readouterr().out, flush=True)
    assert rc == 0
    (st,) = json.loads(out.read_text())["module"]["steps"]
    assert [c["variant"] for c in st["candidates"]] == [0, 1, 2, 3, 4]
    chosen = [c for c in st["candidates"] if c["variant"] == st["chosen"]][0]
    assert chosen["admissible"] and chosen["certificate"]["identity"]["certified"]


def test_module_document_dynamic_extent(tmp_path):
    # The legacy 1-D form's extent is the run's element count: the document
    # needs --elements, which then sizes every dynamic buffer.
    from mlk2_amd import fixtures as fx
    km = fx.config1_module(n=1)
    km.nodes[2].end = -1
    for b in km.buffers:
        b.elements = -1
        b.dims = []
    doc = tmp_path / "dyn.json"
    doc.write_text(km.to_json())
    with pytest.raises(at.UsageError):
        at.config_case("module", at.parse_args([f"--module={doc}"]))
    _, mod, arrays = at.config_case("module", at.parse_args([f"--module={doc}", "--elements=5000"]))
    assert [a.size for a in arrays] == [5000]
    assert all(b.elements == 5000 for b in mod.buffers)
