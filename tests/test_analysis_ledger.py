"""The analysis cache and the measurement ledger (the reference's
packages/tensorlib/src/pdum/tl/analysis.py, pinned the way its
tests/test_analysis.py and conformance/test_fusion_triton.py:87-117 pin it):
content keys, fact composition, the warmth law, JSON-only measurements and a
ledger that round-trips, so nothing keyed identically is measured twice."""

import json

import numpy as np
import pytest

from pdum_dsl_amd.tl import analysis as A
from pdum_dsl_amd.tl import fusion, zoo


@pytest.fixture(autouse=True)
def _cold():
    A.clear(ledger_too=True)
    yield
    A.clear(ledger_too=True)


def test_a_fact_is_computed_once_per_key_and_keys_follow_content():
    calls = []

    @A.defanalysis("t.square", 1)
    def square(x, *, scale=1.0):
        calls.append(x)
        return float(np.sum(x * x)) * scale

    a = np.arange(4.0)
    f1 = square(a)
    f2 = square(a.copy())  # same content, different object: a hit
    assert f1 is f2 and len(calls) == 1 and f1.value == 14.0
    assert square(a, scale=2.0).key != f1.key  # parameters are part of the key
    assert square(a + 1).key != f1.key  # so is the content
    assert f1.analysis == "t.square@v1"
    bumped = A.Analysis("t.square", 2, square.fn)  # a new version is a new key
    assert bumped(a).key != f1.key


def test_a_fact_input_contributes_its_key_and_unwraps_its_value():
    @A.defanalysis("t.base", 1)
    def base(n):
        return list(range(n))

    seen = []

    @A.defanalysis("t.total", 1)
    def total(xs):
        seen.append(xs)
        return sum(xs)

    b = base(5)
    t = total(b)
    assert seen == [[0, 1, 2, 3, 4]] and t.value == 10
    with A.no_reanalysis():  # the whole chain is warm
        assert total(base(5)).key == t.key


def test_no_reanalysis_raises_on_a_miss_and_allows_hits():
    @A.defanalysis("t.id", 1)
    def ident(x):
        return x

    ident(3)
    with A.no_reanalysis():
        ident(3)
        with pytest.raises(A.Reanalysis, match="t.id@v1"):
            ident(4)


def test_unkeyable_inputs_refuse():
    @A.defanalysis("t.any", 1)
    def anyf(x):
        return 0

    with pytest.raises(TypeError, match="content-keyable"):
        anyf(object())


def test_measurements_are_json_records_and_the_ledger_round_trips(tmp_path):
    laps = []

    @A.defanalysis("t.ms", 1, ledger=True)
    def ms(region, *, machine):
        laps.append(machine)
        return {"ms": 1.5, "shape": (2, 3)}  # a tuple normalizes to a JSON list

    @A.defanalysis("t.bad", 1, ledger=True)
    def bad(*, machine):
        return object()

    region = zoo.row_softmax(rows=4, cols=8).region
    f = ms(region, machine="gfx950")
    assert f.value == {"ms": 1.5, "shape": [2, 3]}
    with pytest.raises(TypeError, match="plain data"):
        bad(machine="gfx950")
    path = tmp_path / "ledger.jsonl"
    assert A.save_ledger(path) == 1
    lines = path.read_text().splitlines()
    assert len(lines) == 2 and json.loads(lines[1]) == {"key": f.key, "analysis": "t.ms@v1", "value": f.value}
    assert [p.name for p in tmp_path.iterdir()] == ["ledger.jsonl"]  # saved by rename: no partial file left
    A.clear(ledger_too=True)
    assert A.load_ledger(path) == 1
    with A.no_reanalysis():  # a reloaded measurement is a hit: never measured again
        again = ms(region, machine="gfx950")
    assert again.value == f.value and laps == ["gfx950"]
    assert ms(region, machine="gfx942").key != f.key  # the machine is part of the key


def test_a_warm_replan_certifies_nothing():
    """Certification is a cached fact (fusion.py:696-715): the second plan of
    the same region performs zero analysis."""
    subj = zoo.attention(T=8, E=4, OD=4)
    first = fusion.plan_region(subj.region)
    misses = A.misses()
    with A.no_reanalysis():
        again = fusion.plan_region(subj.region)
    assert A.misses() == misses
    assert again.groups[0].certificate == first.groups[0].certificate


def test_keys_are_typed_and_sets_are_order_free():
    @A.defanalysis("t.k", 1)
    def k(x):
        return 0

    keys = {k(x).key for x in (1, 1.0, True, "1", (1,), None)}
    assert len(keys) == 6  # no two differently typed inputs share a key
    assert k((1, 2)).key == k([1, 2]).key  # sequences are data: a tuple and a list of the same items agree
    assert k({3, 1, 2}).key == k({2, 3, 1}).key and k({"a": 1, "b": 2}).key == k({"b": 2, "a": 1}).key
    a = np.arange(6.0)
    assert k(a.reshape(2, 3)).key != k(a.reshape(3, 2)).key != k(a).key  # shape is part of an array's key
    assert k(a.astype(np.float32)).key != k(a).key


def test_a_file_that_is_not_a_ledger_refuses(tmp_path):
    bad = tmp_path / "other.json"
    bad.write_text(json.dumps({"some": "thing"}))
    with pytest.raises(ValueError, match="not a measurement ledger"):
        A.load_ledger(bad)
    torn = tmp_path / "torn.jsonl"
    torn.write_text(json.dumps({"ledger": "pdum_dsl_amd.measurements", "format": 1}) + "\n" + json.dumps({"key": "k"}))
    with pytest.raises(ValueError, match="exactly key, analysis and value"):
        A.load_ledger(torn)


def test_loading_keeps_a_measurement_taken_in_this_session(tmp_path):
    @A.defanalysis("t.lap", 1, ledger=True)
    def lap(*, machine):
        return {"ms": len(machine)}

    first = lap(machine="gfx950")
    path = tmp_path / "l.jsonl"
    A.save_ledger(path)
    rows = path.read_text().splitlines()
    rec = json.loads(rows[1])
    rec["value"] = {"ms": 99}
    path.write_text(rows[0] + "\n" + json.dumps(rec) + "\n")
    assert A.load_ledger(path) == 1
    assert lap(machine="gfx950").value == first.value == {"ms": 6}


def test_the_jit_counters_read_without_a_device():
    """measure.jit_stats reads the library's host-side counters (no GPU call):
    the warmth guard of the timed loops compares them around the loop."""
    from pdum_dsl_amd import measure as M

    st = M.jit_stats()
    assert set(st) == {"compiled", "launches", "failures"} and all(v >= 0 for v in st.values())
    with M.no_compiles("nothing runs"):
        pass
