"""The CPU oracle reproduces the committed decode-step golden fixtures
(``tests/golden/decode_*.json``, written by ``tests/golden/make_golden.py``):
greedy tokens per step and digests of the logits, resident rows and K/V pages.
The GPU suite checks the HIP decoder against the same files."""
import json
import os

import pytest

from golden.make_golden import CASES, run_oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("case", sorted(CASES))
def test_oracle_reproduces_golden_fixture(case):
    with open(os.path.join(HERE, f"decode_{case}.json")) as f:
        rec = json.load(f)
    assert rec["oracle"] == run_oracle(case)
