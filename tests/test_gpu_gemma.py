"""Gemma3-270M text encoder through the Node host (run_gemma.js -> N-API addon -> C ABI ->
HIP) against the oracle's restatement of tools/reference.py gemma_encode and against that
function's own outputs (tests/golden/gemma_encode.npz), on seeded real-architecture bf16
weights (17 of 18 layers, hidden 640, 4 query heads and 1 K/V head of 256, MLP 2048).
The bf16 linears run fp16 matrix-core products with fp32 accumulation; tolerance 1e-2
(max|d|/max|ref| and rel-L2) for the 17-layer stack, as for the full DiT pass.
"""

import json
import os

import numpy as np
import pytest
import torch

import gemma_fixture as G
from conftest import assert_close

pytestmark = pytest.mark.gpu
TOL_ENCODE = 1e-2
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemma_encode.npz")


@pytest.fixture(scope="module")
def weights_file(tmp_path_factory):
    z = np.load(GOLDEN, allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    d = tmp_path_factory.mktemp("gemma")
    tensors = G.make_weights(seed=meta["weight_seed"])
    path = str(d / "gemma3_bf16.safetensors")
    G.save_weights(tensors, path)
    print(f"[gemma] wrote {os.path.getsize(path) / 2**20:.0f} MiB of seeded weights", flush=True)
    return tensors, path, d, z


def _encode(weights_file, name, ids):
    _, path, d, _ = weights_file
    idf = str(d / f"ids_{name}.json")
    with open(idf, "w") as f:
        json.dump(ids, f)
    out = str(d / f"h_{name}.f32")
    G.run_node(["--weights", path, "--ids", idf, "--out", out])
    return torch.from_numpy(np.fromfile(out, dtype=np.float32).reshape(len(ids), 640))


@pytest.mark.parametrize("case", ["one", "short", "ragged"])
def test_gemma_encode_matches_reference_golden(weights_file, case):
    z = weights_file[3]
    ids = [int(i) for i in z[f"{case}.ids"]]
    got = _encode(weights_file, case, ids)
    assert_close(got, torch.from_numpy(z[f"{case}.out"]), TOL_ENCODE, f"gemma encode {case} (L={len(ids)}) vs golden")


def test_gemma_encode_full_prompt_matches_oracle(weights_file):
    """256 tokens, the longest prompt the pipeline encodes (app/tokenizer.js:11 caps it)."""
    tensors = weights_file[0]
    ids = G.make_ids(256, seed=44)
    got = _encode(weights_file, "full", ids)
    ref = G.oracle_encode(tensors, ids, torch.float32)
    assert_close(got, ref, TOL_ENCODE, "gemma encode 256 tokens vs oracle")


def test_gemma_graph_replays_match_eager(weights_file):
    """A recorded encode (HIP graph, GPU.capture) replayed 4 times, alternating two id sets,
    with an eager encode on the same pooled buffers between replays: every replay equals the
    eager encode of the same ids bit for bit (same kernels, same inputs, deterministic
    reductions)."""
    _, path, d, _ = weights_file
    ids = G.make_ids(37, seed=45)
    idf = str(d / "ids_graph.json")
    with open(idf, "w") as f:
        json.dump(ids, f)
    rep = G.run_node(["--weights", path, "--ids", idf, "--graph-check", "4"])
    checks = rep["graph_check"]
    assert [c["ids"] for c in checks] == [0, 1, 0, 1]
    assert all(c["max_abs_diff"] == 0.0 for c in checks), checks


def test_gemma_graph_output_matches_golden(weights_file):
    """--out from a graph replay (GPU.capture) against the reference's own outputs."""
    _, path, d, z = weights_file
    ids = [int(i) for i in z["short.ids"]]
    idf = str(d / "ids_graph_short.json")
    with open(idf, "w") as f:
        json.dump(ids, f)
    out = str(d / "h_graph_short.f32")
    rep = G.run_node(["--weights", path, "--ids", idf, "--graph", "--out", out])
    assert rep["graph"] is True
    got = torch.from_numpy(np.fromfile(out, dtype=np.float32).reshape(len(ids), 640))
    assert_close(got, torch.from_numpy(z["short.out"]), TOL_ENCODE, "gemma graph replay (short) vs golden")
