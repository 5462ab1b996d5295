"""The synthetic benchmark inputs are pinned by sha256 (tests/golden/input_hashes.json,
written by tests/golden/make_input_hashes.py): the generator in workloads.py must keep
producing byte-identical bf16 tensors for configs 1-4."""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

from make_input_hashes import hashes  # noqa: E402


def test_input_hashes_match_fixture():
    with open(os.path.join(HERE, "golden", "input_hashes.json")) as f:
        want = json.load(f)
    assert hashes() == want
