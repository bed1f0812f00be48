"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_fixtures.py).

CPU: the oracle still reproduces every fixture bit for bit. GPU: the library matches the
fixtures' fp64 results to the parity bar (out max-abs 2e-3, lse 1e-4 + 1e-4 |ref|)."""
import glob
import os

import numpy as np
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

FIXTURES = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))
IDS = [os.path.basename(f)[:-4] for f in FIXTURES]


def load(path):
    z = np.load(path)  # plain arrays only; allow_pickle stays False
    bt = inputs.Batch(list(z["lens"]), int(z["Hq"]), int(z["Hkv"]), z["indptr"], z["indices"], z["last"],
                      int(z["k"].shape[0]), 0, z["q"].view(np.float16), z["k"].view(np.float16),
                      z["v"].view(np.float16))
    return bt, z


def test_fixtures_present():
    assert len(FIXTURES) >= 5


@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_oracle_reproduces_fixture(path, oracle_lib):
    bt, z = load(path)
    o, l = oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv)
    assert np.array_equal(o, z["out"]) and np.array_equal(l, z["lse"])
    po, pl = oracle.partials(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv,
                             int(z["num_chunks"]), int(z["chunk_tokens"]))
    assert np.array_equal(po, z["part_o"]) and np.array_equal(pl, z["part_lse"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_library_matches_fixture(path):
    import _gpu
    bt, z = load(path)
    db = _gpu.DeviceBatch(bt)
    for wg in (0, 1, 5):
        o, l, _ = _gpu.run_plan(db, wg)
        check_out(o, z["out"], tag=f"plan W={wg}")
        check_lse(l, z["lse"], tag=f"plan W={wg}")
    o, l, _ = _gpu.run_uniform(db, int(z["num_chunks"]))
    check_out(o, z["out"], tag="uniform")
    check_lse(l, z["lse"], tag="uniform")
    nc, ct = int(z["num_chunks"]), int(z["chunk_tokens"])
    po, pl = _gpu.run_partials(db, nc, ct)
    check_out(po, z["part_o"], tag="partials")
    check_lse(pl, z["part_lse"], tag="partials")
    if "cascade" in path:
        o, l, info = _gpu.run_cascade(db, min_prefix=16)
        assert info.use == 1
        check_out(o, z["out"], tag="cascade")
        check_lse(l, z["lse"], tag="cascade")
