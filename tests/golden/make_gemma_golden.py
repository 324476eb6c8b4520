"""Writes tests/golden/gemma_encode.npz from the reference implementation itself.

Run in the build container, where the reference is mounted read-only:
    python tests/golden/make_gemma_golden.py [/root/reference]

It imports the reference's Gemma3-270M text encoder (tools/reference.py: gemma_encode, the
hidden state after 17 of 18 layers with the final norm) and drives it with the seeded bf16
weights of tests/gemma_fixture.py (full layer sizes, a 64-row embedding table) on three token
sequences, storing the ids, a weight checksum and the reference's fp32 outputs. Only data is
written; nothing from the reference's sources is copied.
"""

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import gemma_fixture as G  # noqa: E402

WEIGHT_SEED = 5
CASES = [("one", 1, 31), ("short", 12, 32), ("ragged", 37, 33)]  # name, length, id seed


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "tools"))
    import reference as R

    torch.set_grad_enabled(False)
    tensors = G.make_weights(seed=WEIGHT_SEED)

    class Weights:
        """Duck-typed tools/reference.py Weights over in-memory bf16 tensors."""

        def has(self, name):
            return name in tensors

        def __call__(self, name):
            return tensors[name].float()

    out = {}
    meta = {"weight_seed": WEIGHT_SEED, "bf16_sum": sum(float(t.double().sum()) for t in tensors.values()),
            "count": len(tensors), "cases": []}
    for name, L, seed in CASES:
        ids = G.make_ids(L, seed=seed)
        y = R.gemma_encode(Weights(), ids)
        out[f"{name}.ids"] = np.asarray(ids, dtype=np.int32)
        out[f"{name}.out"] = y.float().numpy()
        meta["cases"].append({"name": name, "length": L, "id_seed": seed})
        print(f"{name}: L={L} |y| {float(y.norm()):.4f}", flush=True)
    out["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    path = os.path.join(HERE, "gemma_encode.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
