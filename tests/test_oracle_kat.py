"""The C oracle against the reference's own SIEVE known-answer tests
(test/test_sieve_oracle.py:24-83, transcribed in tests/golden/reference_kats.json)."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as orc

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def _ext_marker_to_slot(s, padded):
    """Reference oracle marker -2-off <-> kernel contract padded+off (xds_decode.py:248-250)."""
    return padded + (-s - 2) if s <= -2 else s


def _run_case(case):
    top_k = max([len(u["topk"]) for u in case.get("updates", [])] + [1])
    st = orc.SieveState(1, case["num_reqs"], case["dbs"], top_k)
    for r in range(case["num_reqs"]):
        st.admit(r, case["prefill"])
    results = []
    for u in case.get("updates", []):
        topk = np.array([u["topk"]], dtype=np.int32)
        slots, miss = st.update(0, topk, [u["req"]], [u["seq_len"]], 1)
        results.append((u, slots[0].tolist(), miss[0].tolist()))
    return st, results


@pytest.mark.parametrize("case", [c for c in KATS["sieve"] if "updates" in c], ids=lambda c: c["name"])
def test_sieve_kat(case):
    st, results = _run_case(case)
    for u, slots, miss in results:
        if "slots" not in u:
            continue
        assert miss == u["miss"], (case["name"], u)
        assert slots == [_ext_marker_to_slot(s, st.padded) for s in u["slots"]], (case["name"], u)
    assert orc.get_error() == 0


def test_ht_churn_consistency():
    case = next(c for c in KATS["sieve"] if c["name"] == "ht_churn_consistency")
    ch = case["churn"]
    st = orc.SieveState(1, 1, case["dbs"], 1)
    st.admit(0, case["prefill"])
    for i in range(ch["count"]):
        slots, miss = st.update(0, np.array([[ch["first_token"] - i]], dtype=np.int32), [0], [ch["seq_len"]], 1)
        assert miss[0, 0] == 1
    tok = st.tokens[0, 0]
    resident = tok[: case["dbs"]]
    assert (resident >= 0).sum() == ch["resident_after"]
    assert len(set(resident.tolist())) == ch["resident_after"]
    ht = st.ht[0, 0]
    assert (ht != 0).sum() == ch["resident_after"]
    for s, t in enumerate(resident.tolist()):
        assert orc.ht_find(ht, tok, t) == s


def test_ext_marker_equivalence():
    """F6: the reference oracle marks decode-extension slots -2-off while the kernel
    contract writes padded+off; the driver's norm maps the former to the latter."""
    padded = 16
    for off in range(5):
        assert _ext_marker_to_slot(-2 - off, padded) == padded + off
    assert _ext_marker_to_slot(-1, padded) == -1
    assert _ext_marker_to_slot(7, padded) == 7
