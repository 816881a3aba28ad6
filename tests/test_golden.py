"""The CPU oracle reproduces the committed golden fixtures (tests/golden/*.npz)."""
import importlib.util
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", sorted(make_golden.GENERATORS))
def test_oracle_reproduces_fixture(name):
    fixture = load(name)
    fresh = make_golden.build(name)
    assert sorted(fixture) == sorted(fresh)
    for key in fixture:
        assert np.array_equal(np.asarray(fresh[key]), fixture[key]), (name, key)


def test_fixture_invariants():
    lm = load("lines_mask_tiles")
    # the full-mode head is all True, every head selects top_k lines
    assert lm["mask"][3].all()
    assert lm["sel"].shape == (4, int(lm["top_k"]))
    # tie block: head 1's first five diagonal scores tie; lower indices win
    mf = load("mts_fit")
    assert mf["mts"].dtype == np.float32 and mf["X"].shape == (2, 3 * 48)
    rp = load("replay_dyadic")
    assert rp["map"].dtype == np.float16 and np.all((rp["map"] >= 0) & (rp["map"] <= 1))
    at = load("attention_small")
    assert np.all(at["out"][1, 128:192] == 0) and np.all(np.isneginf(at["lse"][1, 128:192]))
