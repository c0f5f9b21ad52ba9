"""The golden fixtures still describe the models the synthetic generator makes: same weights.bin
(sha256) and same prompt for every case, so the GPU parity tests compare against the right answer."""
import json
import sys
from functools import lru_cache

import numpy as np
import pytest

from test_gpu_golden import GOLDEN, fixture, synth

sys.path.insert(0, str(GOLDEN))
import make_golden as golden_cases  # noqa: E402


@lru_cache(maxsize=2)
def model_hash(case_json: str):
    case = json.loads(case_json)
    index, buf = synth(case)
    return golden_cases.weights_hash(buf), json.loads(index)["config"]["vocab"]


def case_of(g):
    case = json.loads(str(g["case"]))
    key = json.dumps({k: case[k] for k in ("config", "body", "head", "group", "seed")}, sort_keys=True)
    return case, key


@pytest.mark.parametrize("name", ["c1", "c2", "c2_long", "small_long"])
def test_fixture_matches_generator(name):
    if not (GOLDEN / f"{name}_greedy.npz").exists():
        pytest.skip(f"{name} fixture not generated")
    g = fixture(name)
    case, key = case_of(g)
    assert case == {**golden_cases.CASES[name]}
    sha, vocab = model_hash(key)
    assert sha == str(g["weights_sha256"])
    assert np.array_equal(golden_cases.prompt_ids(case, vocab), g["prompt"])
    assert g["ids"].shape == (case["steps"],) and g["margin"].shape == (case["steps"] + 1,)
    # the sampled logits start with the 16 largest, so their argmax is the greedy pick
    assert int(g["logit_idx"][0][np.argmax(g["logit_val"][0])]) == int(g["ids"][0])


def test_batch_rows_fixture_matches_generator():
    g = fixture("c5_rows")
    case, key = case_of(g)
    assert case == {**golden_cases.CASES["c5_rows"]}
    sha, vocab = model_hash(key)
    assert sha == str(g["weights_sha256"])
    assert np.array_equal(golden_cases.prompt_ids(case, vocab), g["prompt"])
    assert list(g["plen"]) == case["prompt"]
    assert g["ids"].shape == (3, case["steps"]) and g["margin"].shape == (3, case["steps"] + 1)
    for r in range(3):
        assert int(g["logit_idx"][r, 0][np.argmax(g["logit_val"][r, 0])]) == int(g["ids"][r, 0])
