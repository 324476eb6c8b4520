"""Pins the oracle's LoRA merge (tools/reference.py:62-95: w + strength * alpha / r * B A on
access, PEFT and kohya names) to golden vectors written by the reference itself
(tests/golden/make_lora_golden.py loads the seeded weights and LoRA files with the reference's
own Weights class): the DiT x0 with a LoRA on int8 block linears, the GLU linear, a text-refine
linear and bf16 linears, and the Gemma3 encoding with a LoRA on slices of its stacked q/k/v
and gate/up weights."""

import json
import os

import numpy as np
import pytest
import torch

import dit_fixture as F
import gemma_fixture as G
from conftest import assert_close

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "lora_composition.npz")


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN, allow_pickle=False)
    return z, json.loads(bytes(z["meta"]).decode())


def test_dit_lora_matches_reference(golden):
    z, meta = golden
    c = meta["dit_case"]
    tensors = F.make_weights(seed=meta["weight_seed"], I=meta["mlp_width"])
    lora = F.make_lora(seed=meta["lora_seed"], I=meta["mlp_width"])
    inp = F.make_inputs(c["h"], c["w"], c["T"], seed=c["input_seed"], zero_weight_tokens=tuple(c["zero_weight_tokens"]))
    got = F.oracle_forward(tensors, inp, dtype=torch.float32, loras=[(lora, meta["strength"])])
    assert_close(got, torch.from_numpy(z["dit.x0"]), 0.0, "DiT x0 with LoRA (fp32, bit-exact)")
    assert c["rel_change"] > 0.05  # the LoRA moves x0 well beyond the pass tolerance


def test_gemma_lora_matches_reference(golden):
    z, meta = golden
    t = meta["te"]
    tensors = G.make_weights(seed=t["weight_seed"])
    lora = G.make_te_lora(seed=t["lora_seed"])
    ids = [int(i) for i in z["te.ids"]]
    assert ids == G.make_ids(t["ids"][0], seed=t["ids"][1])
    import oracle.nanosaur2_oracle as O

    W = O.TensorWeights(tensors, torch.float64, loras=[(lora, t["strength"])])
    with torch.no_grad():
        got = O.gemma_encode(W, ids, torch.float64)
    assert_close(got.float(), torch.from_numpy(z["te.out"]), 1e-5, "Gemma3 encoding with LoRA")
    assert t["rel_change"] > 0.05
