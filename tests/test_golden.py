"""The CPU oracle against the committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py): caches and T-rounded outputs bit for bit, float64 outputs to
1e-12 relative.  A change to the oracle's arithmetic shows up here first."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import _oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
from make_golden import load  # noqa: E402

FIXTURES = sorted(GOLDEN.glob("*.npz"))


def test_fixtures_present():
    assert len(FIXTURES) >= 5


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: p.stem)
def test_oracle_reproduces_golden(path):
    case, exp = load(path)
    ref, ref_t, kc, vc = orc.paged_attention_op(case)
    assert np.array_equal(kc, exp["key_cache"])
    assert np.array_equal(vc, exp["value_cache"])
    assert np.array_equal(ref_t, exp["output_t"])
    assert orc.rel_l2(ref, exp["output_f64"]) <= 1e-12
