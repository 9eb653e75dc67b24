"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_fixtures.py)
against the oracle: the inputs regenerated from each fixture's seed hash to the stored
value, and the oracle reproduces every stored result exactly -- block tables, table
lengths, free lists, pool hashes and both attention outputs. A change to the oracle's
append, rollback or attention arithmetic fails here."""
import os

import numpy as np

from tests.golden import make_fixtures as F

GOLDEN = os.path.dirname(F.__file__)


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_config1_tiny_oracle_matches_fixture():
    fx = _load("config1_tiny.npz")
    g, x = F.config1_inputs(int(fx["seed"]))
    assert F.sha(x["table"], x["free"], x["k"], x["v"], x["q"], x["k_new"], x["v_new"]) == \
        str(fx["input_sha"])
    e = F.config1_expected(g, x)
    for k in ("status", "tables", "table_lens", "free_list", "out_ref", "out_exact"):
        np.testing.assert_array_equal(e[k], fx[k], err_msg=k)
    assert e["k_sha"] == str(fx["k_sha"]) and e["v_sha"] == str(fx["v_sha"])
    # the append took the back of the LIFO free list for the new (5th) block
    assert fx["table_lens"][0] == 5 and fx["tables"][0, 4] == x["free"][-1]


def test_config5_tiny_oracle_matches_fixture():
    fx = _load("config5_tiny.npz")
    g, x = F.config5_inputs(int(fx["seed"]))
    assert F.sha(*F.config5_input_arrays(x)) == str(fx["input_sha"])
    e = F.config5_expected(g, x)
    for k in ("status", "tables", "table_lens", "free_list", "mtp_ref", "mtp_exact",
              "verify_ref", "verify_exact", "final_pos", "k_sha", "v_sha"):
        np.testing.assert_array_equal(e[k], fx[k], err_msg=k)
