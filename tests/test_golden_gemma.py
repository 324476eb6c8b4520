"""Pins the oracle's Gemma3-270M text encoder to golden vectors written by the reference
implementation itself (tests/golden/make_gemma_golden.py runs tools/reference.py
gemma_encode): norm weights stored as w - 1, the theta schedule of the split-half RoPE,
grouped causal attention, the GELU(tanh)-gated MLP and the final norm after layer 17."""

import json
import os

import numpy as np
import pytest
import torch

import gemma_fixture as G
from conftest import assert_close

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemma_encode.npz")


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN, allow_pickle=False)
    return z, json.loads(bytes(z["meta"]).decode())


@pytest.fixture(scope="module")
def weights(golden):
    _, meta = golden
    t = G.make_weights(seed=meta["weight_seed"])
    bf = sum(float(v.double().sum()) for v in t.values())
    assert len(t) == meta["count"] and abs(bf - meta["bf16_sum"]) < 1e-9, "weight generator drifted"
    return t


@pytest.mark.parametrize("case", ["one", "short", "ragged"])
def test_gemma_encode_matches_reference(golden, weights, case):
    z, _ = golden
    ids = [int(i) for i in z[f"{case}.ids"]]
    assert ids == G.make_ids(len(ids), seed={"one": 31, "short": 32, "ragged": 33}[case])
    got = G.oracle_encode(weights, ids, torch.float64)
    assert_close(got.float(), torch.from_numpy(z[f"{case}.out"]), 1e-5, f"gemma {case}")


def test_gemma_encode_is_causal(weights):
    """Appending tokens leaves the earlier rows of the encoding unchanged."""
    ids = G.make_ids(9, seed=40)
    a = G.oracle_encode(weights, ids[:5], torch.float64)
    b = G.oracle_encode(weights, ids, torch.float64)
    assert torch.allclose(a, b[:5], atol=1e-9, rtol=0)
