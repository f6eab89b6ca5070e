"""CPU checks of the committed golden fixtures (tests/golden/).

* every fixture file matches the sha256 in the manifest;
* the oracle regenerates every fixture bit for bit from its seeds (a change to
  the oracle that moves any expected value fails here);
* each fixture's expected outputs agree with an independent float64 numpy
  formulation of the reference formula within the op's tolerance, or with numpy
  indexing bit for bit (gather, KV appends, widening);
* the reference's own known answers held by two fixtures
  (tests/test_softmax.cu:88-106, tests/test_kvcache.cu:63-68)."""
import hashlib
import json

import numpy as np
import pytest

from golden import make_golden as mg

NAMES = mg.names()


def test_manifest_lists_every_case():
    assert set(NAMES) == set(mg.CASES)
    man = json.loads(mg.MANIFEST.read_text())
    for name in NAMES:
        assert man["fixtures"][name]["params"]["tol"] in (*mg.TOL, "attention")


@pytest.mark.parametrize("name", NAMES)
def test_fixture_sha256(name):
    ent = json.loads(mg.MANIFEST.read_text())["fixtures"][name]
    assert hashlib.sha256((mg.HERE / ent["file"]).read_bytes()).hexdigest() == ent["sha256"]


@pytest.mark.parametrize("name", NAMES)
def test_oracle_regenerates_fixture(name):
    params, arrays = mg.load(name)
    p2, a2 = mg.CASES[name]()
    assert json.loads(json.dumps(p2)) == params
    assert sorted(a2) == sorted(arrays)
    for k, v in arrays.items():
        w = np.asarray(a2[k])
        assert w.dtype == v.dtype and w.shape == v.shape, (name, k)
        assert w.tobytes() == v.tobytes(), f"{name}: {k} differs from the committed fixture"


@pytest.mark.parametrize("name", NAMES)
def test_fixture_matches_float64_formulation(name):
    params, arrays = mg.load(name)
    mg.independent_check(params, arrays)


def test_reference_known_answers():
    _, a = mg.load("softmax_f32_reftest")
    # inputs are the first rows of srand(7) U(-2,2): rand()/RAND_MAX*4-2
    assert a["in_x"].shape == (4, 2048) and np.abs(a["in_x"]).max() <= 2.0
    assert np.abs(a["want_out"] - a["want_reftest_cpu"]).max() < 1e-5
    _, a = mg.load("kv_append_f32_readback")
    assert a["want_k_cache"][0, 7, 0, 0] == np.float32(7.0)
    assert np.all(a["want_v_cache"][:, 7] == np.float32(-7.0))


def test_independent_check_catches_a_planted_slip():
    # a one-ulp slip in one expected value of an exact op, and a sign slip in a
    # rotated pair, must both be rejected
    params, a = mg.load("embed_f16")
    a = dict(a)
    a["want_out"] = a["want_out"].copy()
    a["want_out"][0, 5] ^= 1
    with pytest.raises(AssertionError):
        mg.independent_check(params, a)
    params, a = mg.load("rope_f32_half")
    a = dict(a)
    a["want_q"] = a["want_q"].copy()
    a["want_q"][5, 40] = -a["want_q"][5, 40]
    with pytest.raises(AssertionError):
        mg.independent_check(params, a)
