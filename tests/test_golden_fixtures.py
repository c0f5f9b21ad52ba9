"""The golden fixtures still describe the models the synthetic generator makes: same weights.bin
(sha256) and same prompt for every case, so the GPU parity tests compare against the right answer."""
import json
import sys

import numpy as np
import pytest

from test_gpu_golden import GOLDEN, fixture, synth

sys.path.insert(0, str(GOLDEN))
import make_golden as golden_cases  # noqa: E402


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_fixture_matches_generator(name):
    g = fixture(name)
    case = json.loads(str(g["case"]))
    index, buf = synth(case)
    assert golden_cases.weights_hash(buf) == str(g["weights_sha256"])
    vocab = json.loads(index)["config"]["vocab"]
    assert np.array_equal(golden_cases.prompt_ids(case, vocab), g["prompt"])
    assert g["ids"].shape == (case["steps"],) and g["margin"].shape == (case["steps"] + 1,)
    # the sampled logits start with the 16 largest, so their argmax is the greedy pick
    assert int(g["logit_idx"][0][np.argmax(g["logit_val"][0])]) == int(g["ids"][0])
