"""The CPU oracle reproduces every committed golden digest
(tests/golden/golden.json, written by tests/golden/make_golden.py): a rebuild
of the oracle (compiler, flags) that changed any output bit fails here before
any GPU run compares against it."""
import json
import os

import pytest

import cases

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "golden.json")))["cases"]


@pytest.mark.parametrize("name", sorted(GOLDEN))
def test_oracle_matches_golden_digest(ora, name):
    build, oracle_fn = cases.golden_cases()[name]
    inp, meta = build()
    assert cases.digest(oracle_fn(ora, inp, meta)) == GOLDEN[name]["sha256"], name
