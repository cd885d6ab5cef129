"""The oracle against its committed golden fixtures (tests/golden/).

The reference holds no vectors of its own, so the fixtures written by
tests/golden/make_golden.py (seeded inputs + the oracle's float64 outputs)
guard the oracle's restatement of SFA.py:359-853, 964-970 against drift: the
file must match its recorded sha256, the recorded seeds must regenerate the
stored inputs, and the oracle must reproduce every stored output."""
import hashlib
import json
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
sys.path.insert(0, GOLDEN)

import make_golden  # noqa: E402

with open(os.path.join(GOLDEN, "MANIFEST.json")) as f:
    MANIFEST = json.load(f)
NPZ = os.path.join(GOLDEN, MANIFEST["file"])


def _case(name):
    z = np.load(NPZ)  # allow_pickle=False (the default): plain arrays only
    return {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}


def test_fixture_file_matches_manifest():
    with open(NPZ, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == MANIFEST["sha256"]
    assert set(MANIFEST["cases"]) == set(make_golden.CASES)


@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_seeds_regenerate_inputs(name):
    stored = _case(name)
    fresh = make_golden.make_inputs(make_golden.CASES[name])
    for k, a in fresh.items():
        assert np.array_equal(stored[k], a), k


@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_oracle_reproduces_fixture(name):
    stored = _case(name)
    inputs = {k: stored[k] for k in MANIFEST["cases"][name]["inputs"]}
    got = make_golden.oracle_outputs(inputs)
    assert sorted(got) == MANIFEST["cases"][name]["outputs"]
    for k, a in got.items():
        ref = stored[k]
        fin = np.isfinite(ref)
        assert np.array_equal(np.isfinite(a), fin), k
        assert np.allclose(a[fin], ref[fin], rtol=1e-12, atol=1e-12), (k, float(np.abs(a[fin] - ref[fin]).max()))


def test_fixture_detects_a_planted_oracle_mistake():
    """A dropped scale factor in the oracle's input (scale 1 instead of
    1/sqrt(d)) moves every stored output well outside the tolerance."""
    stored = _case("gqa_kvlens_sink_fp32")
    inputs = {k: stored[k] for k in MANIFEST["cases"]["gqa_kvlens_sink_fp32"]["inputs"]}
    inputs["scale"] = np.asarray(1.0)
    got = make_golden.oracle_outputs(inputs)
    assert not np.allclose(got["out"], stored["out"], atol=1e-3)
    assert not np.allclose(got["dq"], stored["dq"], atol=1e-3)
