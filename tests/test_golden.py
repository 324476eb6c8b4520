"""Pins the oracle to golden vectors written by the reference implementation itself
(tests/golden/make_golden.py runs tools/reference.py and tools/quant.py): the DiT
composition (text refine, SPRINT wiring, pooling clamp, masking of zero-weight tokens,
path-drop) and the exact int8 ConvRot quantization."""

import json
import os

import numpy as np
import pytest
import torch

import dit_fixture as F
import oracle.nanosaur2_oracle as O
from conftest import assert_close

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dit_composition.npz")


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN, allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    return z, meta


@pytest.fixture(scope="module")
def weights(golden):
    _, meta = golden
    t = F.make_weights(seed=meta["weight_seed"], I=meta["mlp_width"])
    i8 = sum(int(v.to(torch.int64).sum()) for v in t.values() if v.dtype == torch.int8)
    bf = sum(float(v.double().sum()) for v in t.values() if v.dtype == torch.bfloat16)
    sc = sum(float(v.double().sum()) for n, v in t.items() if n.endswith("weight_scale"))
    c = meta["checksums"]
    assert (i8, len(t)) == (c["int8_sum"], c["count"]), "weight generator drifted from the golden run"
    assert abs(bf - c["bf16_sum"]) < 1e-9 and abs(sc - c["scale_sum"]) < 1e-9
    return t


def test_quantize_matches_reference(golden):
    z, _ = golden
    q, s = O.quantize_int8_convrot(torch.from_numpy(z["quant.w"]))
    assert np.array_equal(q.numpy(), z["quant.q"])
    assert np.array_equal(s.numpy(), z["quant.scale"])
    meta = json.loads(bytes(z["quant.meta"]).decode())
    assert meta["format"] == "int8_tensorwise" and meta["convrot"] is True
    assert json.loads(F.COMFY_QUANT.decode()) == meta


@pytest.mark.parametrize("case", [0, 1])
def test_dit_composition_matches_reference(golden, weights, case):
    z, meta = golden
    c = meta["cases"][case]
    inp = F.make_inputs(c["h"], c["w"], c["T"], seed=c["input_seed"], zero_weight_tokens=c["zero_weight_tokens"])
    assert inp["sigma"] == c["sigma"]
    dit = O.DiT(O.TensorWeights(weights))
    dump = {}
    with torch.no_grad():
        x0 = dit.forward(torch.from_numpy(inp["latent"]), inp["sigma"], torch.from_numpy(inp["context"]),
                         torch.from_numpy(inp["weights"]), path_drop=c["path_drop"], dump=dump)
    name = c["name"]
    for k in ("txt_refined", "cond", "block1"):
        assert_close(dump[k], torch.from_numpy(z[f"{name}.{k}"]), 1e-5, f"oracle {name}.{k} vs reference")
    assert_close(x0, torch.from_numpy(z[f"{name}.x0"]), 1e-5, f"oracle {name}.x0 vs reference")
