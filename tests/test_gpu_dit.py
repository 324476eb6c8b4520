"""Full DiT pass through the Node host (run_dit.js -> N-API addon -> C ABI -> HIP) against the
oracle's restatement of tools/reference.py DiT.forward, on seeded real-architecture weights
(D=1536, 18 blocks, I=4096, int8 ConvRot block linears).

Two bounds on x0 (max|d|/max|ref| and rel-L2): the 1e-2 required of a full 18-block pass, and a
regression bound near the measured error of the fp16-operand path (rel-L2 4.5e-4 to 6.2e-4,
max 6e-4 to 1.3e-3), so that a tenfold loss of precision fails even though it would stay inside
1e-2. The reference's own check harness compares its WebGPU x0 against fp32 PyTorch at a
rel-L2 of 1e-4 (tools/check.js:89-98); that bound is for an fp32 engine, and fp16 MFMA operands
cannot meet it (each rounding is 2^-11 relative).
"""

import os

import numpy as np
import pytest
import torch

import dit_fixture as F
from conftest import assert_close, rel_errors

pytestmark = pytest.mark.gpu
TOL_PASS = 1e-2
REG_REL_L2 = 2e-3   # regression bound, about 3x the measured rel-L2
REG_MAX = 4e-3      # regression bound, about 3x the measured max|d|/max|ref|


def assert_pass(got, ref, what):
    assert_close(got, ref, TOL_PASS, what)
    max_rel, rel_l2 = rel_errors(got, ref)
    assert rel_l2 <= REG_REL_L2 and max_rel <= REG_MAX, \
        f"{what}: precision regression: max_rel {max_rel:.3e} (bound {REG_MAX}), rel_l2 {rel_l2:.3e} (bound {REG_REL_L2})"


@pytest.fixture(scope="module")
def weights_file(tmp_path_factory):
    d = tmp_path_factory.mktemp("dit")
    tensors = F.make_weights(seed=3)
    path = str(d / "dit_int8.safetensors")
    F.save_weights(tensors, path)
    print(f"[dit] wrote {os.path.getsize(path) / 2**20:.0f} MiB of seeded weights", flush=True)
    return tensors, path, d


def _run_case(weights_file, name, h, w, T, *, zero=(), path_drop=False, reference_ops=False, seed=7, extra=()):
    tensors, path, d = weights_file
    inp = F.make_inputs(h, w, T, seed=seed, zero_weight_tokens=zero)
    idir = str(d / f"in_{name}")
    F.write_inputs(inp, idir)
    out = str(d / f"x0_{name}.f32")
    args = ["--weights", path, "--inputs", idir, "--out", out]
    if path_drop:
        args.append("--path-drop")
    if reference_ops:
        args.append("--reference-ops")
    args += list(extra)
    rep = F.run_node(args)
    got = torch.from_numpy(np.fromfile(out, dtype=np.float32).reshape(64, h, w))
    ref = F.oracle_forward(tensors, inp, path_drop=path_drop)
    assert_pass(got, ref, f"DiT pass {name} ({h}x{w}, T={T})")
    return rep


def test_dit_pass_fused(weights_file):
    _run_case(weights_file, "fused", 6, 8, 16)


def test_dit_pass_reference_op_sequence(weights_file):
    """The reference's op sequence (separate headNorm / rotate / glu) on the same ops API."""
    _run_case(weights_file, "refops", 6, 8, 16, reference_ops=True)


def test_dit_pass_masked_token_and_path_drop(weights_file):
    """A zero-weight prompt token (dropped by the host, masked by the reference) and the
    path-drop pass that skips the SPRINT blocks."""
    _run_case(weights_file, "masked", 5, 7, 12, zero=(3,), seed=11)
    _run_case(weights_file, "pathdrop", 5, 7, 12, path_drop=True, seed=12)


def test_dit_pass_cancelled_between_blocks(weights_file):
    """A pass cancelled from onBlock after 5 blocks (the pipeline's cancel, app/pipeline.js:233-247):
    the AbortError propagates after exactly those blocks, every pooled buffer of the pass is back
    in the pool, and the next pass on the same model matches the oracle."""
    rep = _run_case(weights_file, "cancel", 6, 8, 16, extra=["--abort-at", "5"])
    ab = rep["abort"]
    assert ab["error"] == "AbortError" and ab["blocks"] == 5, ab
    assert ab["live_after"] == ab["live_before"], ab


def test_dit_pass_against_reference_golden(tmp_path):
    """The HIP path against x0 written by the reference implementation itself
    (tests/golden/dit_composition.npz; MLP width 256)."""
    import json

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "dit_composition.npz"), allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    tensors = F.make_weights(seed=meta["weight_seed"], I=meta["mlp_width"])
    path = str(tmp_path / "golden_w.safetensors")
    F.save_weights(tensors, path)
    for c in meta["cases"]:
        inp = F.make_inputs(c["h"], c["w"], c["T"], seed=c["input_seed"], zero_weight_tokens=c["zero_weight_tokens"])
        idir = str(tmp_path / c["name"])
        F.write_inputs(inp, idir)
        out = str(tmp_path / f"{c['name']}.f32")
        args = ["--weights", path, "--inputs", idir, "--out", out] + (["--path-drop"] if c["path_drop"] else [])
        F.run_node(args)
        got = torch.from_numpy(np.fromfile(out, dtype=np.float32).reshape(64, c["h"], c["w"]))
        assert_pass(got, torch.from_numpy(z[f"{c['name']}.x0"]), f"HIP pass vs reference golden {c['name']}")


# ------------------------------------------------------------------ the benchmarked size (832x1216)

FULL_H, FULL_W, FULL_T = 76, 52, 256   # 832x1216 image -> 76 x 52 latent = 3952 tokens; 256 prompt tokens


@pytest.fixture(scope="module")
def full_size(weights_file):
    """The workload bench.py times: 76 x 52 latent, 256 prompt tokens with weights U[0.5, 1.5]
    and one zero-weight token (dropped by the host, masked by the reference), so the pass runs
    the 64x128 tiles over 3952 rows, the 66-tile key loop split at the first text tile, the
    split-K text linears and the pool/workspace reuse over 18 blocks. Oracle results are
    cached per path-drop flag."""
    tensors, path, d = weights_file
    inp = F.make_inputs(FULL_H, FULL_W, FULL_T, seed=21, zero_weight_tokens=(37,))
    idir = str(d / "in_full")
    F.write_inputs(inp, idir)
    return {"inp": inp, "dir": idir, "ref": {}}


@pytest.mark.parametrize("mode", ["fused", "reference_ops", "path_drop"])
def test_dit_pass_full_size(weights_file, full_size, mode):
    """x0 of the 832x1216 pass against the oracle's fp32 DiT.forward, at 1e-2 and at the
    regression bound: the fused driver, the reference's op sequence, and the path-drop pass
    (blocks 2-15 skipped)."""
    tensors, path, d = weights_file
    path_drop = mode == "path_drop"
    out = str(d / f"x0_full_{mode}.f32")
    args = ["--weights", path, "--inputs", full_size["dir"], "--out", out]
    if path_drop:
        args.append("--path-drop")
    if mode == "reference_ops":
        args.append("--reference-ops")
    F.run_node(args)
    got = torch.from_numpy(np.fromfile(out, dtype=np.float32).reshape(64, FULL_H, FULL_W))
    if path_drop not in full_size["ref"]:
        full_size["ref"][path_drop] = F.oracle_forward(tensors, full_size["inp"], path_drop=path_drop)
    assert_pass(got, full_size["ref"][path_drop],
                f"DiT pass 832x1216 {mode} ({FULL_H}x{FULL_W}, T={FULL_T}, one zero-weight token)")
