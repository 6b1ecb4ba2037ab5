"""The oracle's window and capacity math against the reference's own C++
contract helpers, built from the reference headers by oracle/Makefile into
oracle/_ref/ (skipped where that build is absent)."""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import pytest

from oracle import kv_oracle as O

REF_BIN = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "ref_contracts"


@pytest.fixture(scope="module")
def ref_rows():
    if not REF_BIN.exists():
        pytest.skip("oracle/_ref/ref_contracts not built (needs /root/reference)")
    out = subprocess.run([str(REF_BIN)], check=True, capture_output=True, text=True).stdout
    return [json.loads(line) for line in out.splitlines()]


def test_causal_limits_and_sliding_starts_match_the_reference_helpers(ref_rows):
    n = 0
    for r in ref_rows:
        if r["kind"] == "causal":
            lo, hi = O.visible_range(r["prefix"] + r["q"], 0)
            assert (lo, hi + 1) == (0, r["limit"]), r
            n += 1
        elif r["kind"] == "sliding":
            lo, _ = O.visible_range(r["prefix"] + r["q"], r["window"])
            assert lo == r["start"], r
            n += 1
    assert n > 10000


def test_ring_capacity_matches_the_reference_contract(ref_rows):
    rows = [r for r in ref_rows if r["kind"] == "capacity"]
    assert len(rows) == 64
    for r in rows:
        assert r["ok"]
        assert O.ring_capacity(r["window"], r["max_q"], r["max_seq"]) == r["capacity"], r
