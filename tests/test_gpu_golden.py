"""The HIP path (operator entry, through the C ABI) against the committed golden fixtures:
key/value pools bit-exact; output rel-L2 <= 2e-3 against the stored T-rounded oracle output
(fp16/bf16) and <= 4e-3 against the stored float64 output."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import _oracle as orc
from pa_cases import run_gpu_op

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
from make_golden import load  # noqa: E402

FIXTURES = sorted(GOLDEN.glob("*.npz"))


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: p.stem)
def test_hip_matches_golden(path):
    case, exp = load(path)
    print(f"golden case {path.stem}", flush=True)
    out, kc, vc = run_gpu_op(case)
    assert np.array_equal(kc, exp["key_cache"]), "key cache differs from the fixture"
    assert np.array_equal(vc, exp["value_cache"]), "value cache differs from the fixture"
    dt = case["dtype"]
    got = orc.decode(out, dt).astype(np.float64)
    err_t = orc.rel_l2(got, orc.decode(exp["output_t"], dt))
    err64 = orc.rel_l2(got, exp["output_f64"])
    assert err_t <= 2e-3, f"rel-L2 vs fixture (T) {err_t:.3e}"
    assert err64 <= 4e-3, f"rel-L2 vs fixture (f64) {err64:.3e}"
